// Shader clock probe: a dependent multiply-add chain (separate mul and add)
// in one wave, timed by clock64() (shader clock) and wall_clock64() (100 MHz),
// giving the shader clock and the cost of a dependent VALU step.
//
//   hipcc -O3 --offload-arch=gfx950 -ffp-contract=off loom_amd/probes/clock_probe.hip -o clock_probe
#include <hip/hip_runtime.h>
#include <cstdio>
__global__ void chain(float *out, unsigned long long *t, int n, float a) {
    float v = a;
    unsigned long long c0 = clock64(), w0 = wall_clock64();
    for (int i = 0; i < n; i++) v = v * 1.0000001f + 0.5f;
    unsigned long long c1 = clock64(), w1 = wall_clock64();
    if (threadIdx.x == 0) { t[0] = c1 - c0; t[1] = w1 - w0; out[blockIdx.x] = v; }
}
int main() {
    float *out; unsigned long long *t, h[2];
    hipMalloc(&out, 4096 * 4); hipMalloc(&t, 16);
    for (int rep = 0; rep < 6; rep++) {
        int n = rep < 3 ? 100000 : 10000000;
        hipLaunchKernelGGL(chain, dim3(1), dim3(64), 0, 0, out, t, n, 1.0f);
        hipMemcpy(h, t, 16, hipMemcpyDeviceToHost);
        printf("n=%d cycles=%llu wall=%llu (x10ns) -> shader clock %.0f MHz, %.2f cycles/op, %.2f ns/op\n",
               n, h[0], h[1], h[0] / (h[1] * 10e-3), (double)h[0] / n, h[1] * 10.0 / n);
    }
    return 0;
}
