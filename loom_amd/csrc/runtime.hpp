// runtime.hpp -- host-side context of libloomhip.
#pragma once

#include "../../include/loomhip.h"
#include "kernels.hpp"

#include <unordered_map>

namespace lh {

constexpr int IOTA_LEN = 1 << 16; // identity pair table (max pairs / vectors per launch)

// Grow-only device buffer.  Reallocation synchronises the compute stream.
struct Scratch {
    void *ptr = nullptr;
    size_t cap = 0;
    int reserve(size_t bytes);
    void release() {
        if (ptr)
            (void)hipFree(ptr);
        ptr = nullptr;
        cap = 0;
    }
};

struct Ctx {
    bool ready = false;
    int device = -1;
    hipStream_t compute = nullptr; // kernels
    hipStream_t copy = nullptr;    // expert-cache host->HBM copies
    const int *iota = nullptr;
    int *sync = nullptr; // SYNC_INTS zero-initialised completion counters
    Scratch act;    // quantized activations for dense matvecs
    Scratch xstage; // seam-call staging
    Scratch ostage;
    std::unordered_map<int, void *> dense_tables;
};

extern Ctx g_ctx;

int fail(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);
int require_ready();
hipStream_t stream_of(void *s);
int upload_weights(int t, const void *host, size_t rows, size_t cols, size_t planes, void **dev);
void clear_weight_cache();
int matvec_dev_impl(int t, float *out, const void *w, const float *x, size_t n, size_t rows,
                    size_t cols, hipStream_t st);
int pick_nt(int n);
// From this many vectors per weight plane on, Q4_K / Q6_K matmuls run on the
// matrix cores (mmq.hip) in groups of up to 32 (dense) or 16 (experts).
constexpr int MMQ_MIN_TOK = 16;
inline bool use_mmq(int t, int cols, int n, int group_tok, bool fused) {
    return n >= MMQ_MIN_TOK && mmq_supported(t, cols, group_tok, fused);
}
// Device group table for n vectors in groups of nt against plane 0 (cached per (n, nt)).
const DmmvGroup *dense_groups(int n, int nt, int *count);
void moe_release_scratch();
// A dense SwiGLU FFN of one plane per tensor (device layout): the shared
// expert of a routed MoE layer.  dense_ffn_add: out[t] (+)= down . swiglu(gate .
// x_t, up . x_t) for n vectors (add: a residual-add epilogue), bit-identical
// to the CPU kernels.
struct DenseFfn {
    int gate_t, up_t, down_t;
    const void *gate, *up, *down; // gate null: none
    size_t ffn;
};
int dense_ffn_check(const DenseFfn &f, size_t dim);
int dense_ffn_add(const DenseFfn &f, const float *x, size_t n, size_t dim, float *out, hipStream_t st, bool add);
// Resolves this device's copy of the no-allocation entry point's fixed scratch.
int moe_noalloc_setup(int device);
// The decode MoE path with its rmsnorm fused into the router launch (x = the
// residual stream); moe_decode_fusable says whether the layer takes it.
// exact: the squares summed in the reference's order (one token), else a tree.
int moe_layer_fused_norm(const loomhip_moe_layer *L, const float *x, const float *norm_w, float eps, size_t n_tok,
                         int combine, float *out, uint32_t *ids_out, bool exact, hipStream_t st);
bool moe_decode_fusable(const loomhip_moe_layer *L, size_t n_tok, bool exact);
// loomhip_moe_layer_dev with, on the batched path, the next rmsnorm of the
// residual row (next) formed in the combine's launch; *next_done says it ran.
int moe_layer_next_norm(const loomhip_moe_layer *L, const float *normed, size_t n_tok, int combine, float *out,
                        uint32_t *ids_out, const NextNorm *next, bool *next_done, hipStream_t st);
// What the MoE layer would decline at n tokens, checked before any launch.
int moe_frame_check(const loomhip_moe_layer *L, size_t n);
// The same checks for a caller that forms acc = routed + shared itself
// (shexp_ok) before adding it to the residual.
int moe_layer_check(const loomhip_moe_layer *L, size_t n, bool shexp_ok);
void ec_release_scratch();
void block_release_cache();
void mla_release();
void seam_release(); // the seam's device K/V cache, frame residual and staging
// The exact rmsnorm (squares summed in order) of n rows into normed.
int rmsnorm_exact_dev(const float *x, int dim, const float *w, float eps, float *normed, size_t n, hipStream_t st);

} // namespace lh
