// Latency calibration probe for the decode kernels' design: duration of an
// empty kernel, of one HBM round trip, of a dependent second load, and of 16
// independent 16-byte loads per lane, at 16..4096 work groups of 256.
//
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         loom_amd/probes/latency_probe.hip -o latency_probe
//   rocprofv3 --kernel-trace --stats --output-format csv -d out -o probe -- ./latency_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>

__global__ void k_empty(float *out) {
    if (threadIdx.x == 0 && blockIdx.x == 1u << 30) out[0] = 1.f;
}

__global__ void k_load1(const float4 *__restrict__ in, float *__restrict__ out, size_t stride) {
    const size_t i = (size_t)blockIdx.x * stride + threadIdx.x;
    float4 v = in[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = v.x + v.y + v.z + v.w;
}

__global__ void k_load_dep2(const float4 *__restrict__ in, const int *__restrict__ idx,
                            float *__restrict__ out, size_t stride) {
    const int j = idx[blockIdx.x];
    const size_t i = (size_t)j * stride + threadIdx.x;
    float4 v = in[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = v.x + v.y + v.z + v.w;
}

// each lane issues N independent 16-byte loads, then sums
template <int N>
__global__ void k_loadN(const float4 *__restrict__ in, float *__restrict__ out, size_t stride) {
    float acc = 0.f;
    float4 v[N];
#pragma unroll
    for (int u = 0; u < N; u++)
        v[u] = in[(size_t)blockIdx.x * stride + u * blockDim.x + threadIdx.x];
#pragma unroll
    for (int u = 0; u < N; u++)
        acc += v[u].x + v[u].y + v[u].z + v[u].w;
    out[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

int main() {
    const size_t big = (size_t)2 << 30; // 2 GiB, defeats MALL when rotated
    float4 *in;
    float *out;
    int *idx;
    hipMalloc(&in, big);
    hipMalloc(&out, 64 << 20);
    hipMalloc(&idx, 4096 * 4);
    hipMemset(in, 0, big);
    std::vector<int> h(4096);
    for (int i = 0; i < 4096; i++) h[i] = (i * 7919) % 4096;
    hipMemcpy(idx, h.data(), 4096 * 4, hipMemcpyHostToDevice);
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    const int R = 200;
    auto run = [&](const char *name, auto launch) {
        for (int i = 0; i < 10; i++) launch(i);
        hipDeviceSynchronize();
        hipEventRecord(a);
        for (int i = 0; i < R; i++) launch(i);
        hipEventRecord(b);
        hipEventSynchronize(b);
        float ms;
        hipEventElapsedTime(&ms, a, b);
        printf("%-28s %8.2f us/launch (back-to-back)\n", name, ms * 1000 / R);
    };
    const size_t n4 = big / 16;
    for (int wgs : {16, 256, 1024, 4096}) {
        char nm[64];
        snprintf(nm, sizeof nm, "empty wgs=%d", wgs);
        run(nm, [&](int) { hipLaunchKernelGGL(k_empty, dim3(wgs), dim3(256), 0, 0, out); });
        snprintf(nm, sizeof nm, "load1 wgs=%d", wgs);
        // rotate the base over 2 GiB so repeats miss the caches
        run(nm, [&](int i) {
            size_t stride = n4 / 4096;
            hipLaunchKernelGGL(k_load1, dim3(wgs), dim3(256), 0, 0, in + (i % 3) * 977, out, stride);
        });
        snprintf(nm, sizeof nm, "load_dep2 wgs=%d", wgs);
        run(nm, [&](int i) {
            size_t stride = n4 / 4096;
            hipLaunchKernelGGL(k_load_dep2, dim3(wgs), dim3(256), 0, 0, in + (i % 3) * 977, idx, out, stride);
        });
        snprintf(nm, sizeof nm, "load16 wgs=%d", wgs);
        run(nm, [&](int i) {
            size_t stride = n4 / 4096;
            hipLaunchKernelGGL(k_loadN<16>, dim3(wgs), dim3(256), 0, 0, in + (i % 3) * 977, out, stride);
        });
    }
    printf("done\n");
    return 0;
}
