// Launchers of the gfx950 kernels (pi_kernels.hip).  All launch on `s` and
// return hipSuccess or the launch error; none synchronizes.
#pragma once

#include <hip/hip_runtime_api.h>

#include "pi_common.h"

// Decode-step state kept in HBM so one captured graph serves every position.
struct pi_state {
    int32_t  pos;     // position of the token being evaluated
    uint32_t tok;     // token being evaluated
    uint32_t n_gen;   // generated ids written so far
    uint32_t i;       // prompt index during prefill
};

enum pi_gemv_mode { PI_GEMV_OUT = 0, PI_GEMV_RESIDUAL = 1, PI_GEMV_SUMS = 2 };

// Up to three matrices of one type and row length that share an activation.
// tile0[m] is the first tile of matrix m in a back-to-back numbering;
// tile0[n..3] hold the total tile count.
struct pi_gemv_set {
    const uint8_t *w[3];
    float *y[3];
    uint32_t rows[3];
    uint32_t tile0[4];
    uint32_t n;
};

hipError_t pi_launch_repack(const uint8_t *src_native, uint8_t *dst, const pi_layout &L, hipStream_t s);

// Q8Act::prepare (quant_int.rs:17-56); x feature-major [k][b].
hipError_t pi_launch_q8(const float *x, uint32_t k, uint32_t b, int8_t *q, float *d, int32_t *sum,
                        hipStream_t s);

// y[r] = 0 + acc (OUT), y[r] = y[r] + (0 + acc) (RESIDUAL), or integer sums (SUMS).
hipError_t pi_launch_gemv(const uint8_t *w, const pi_layout &L, const int8_t *aq, const float *ad,
                          const int32_t *as, float *y, int32_t *sums, int mode, int max_blocks,
                          hipStream_t s);

// One launch over a pi_gemv_set (OUT or RESIDUAL); L gives the common layout.
hipError_t pi_launch_gemv_group(const pi_gemv_set &S, const pi_layout &L, const int8_t *aq, const float *ad,
                                const int32_t *as, int mode, int max_blocks, hipStream_t s);

// Engine::rmsnorm (model.rs:777-823) fused with Q8 quantization of the result;
// `out` (optional) receives the normalized f32 vector.
// neon selects the batch-1 order of the aarch64 build, else the scalar loop.
hipError_t pi_launch_rmsnorm_q8(const float *x, const float *w, uint32_t ne, float eps, float *out,
                                int8_t *q, float *d, int32_t *sum, bool neon, hipStream_t s);

// SwiGLU (model.rs:1111-1115) fused with Q8 quantization.
hipError_t pi_launch_swiglu_q8(const float *gate, const float *up, uint32_t n, int8_t *q, float *d,
                               int32_t *sum, hipStream_t s);

// Embedding row (model.rs:857-869) of the token in st->tok (or `tok` when st == nullptr).
hipError_t pi_launch_embed(const uint8_t *embd_native, uint32_t type, uint32_t ne, uint64_t row_bytes,
                           const pi_state *st, float *x, hipStream_t s);

// RoPE (model.rs:953-979) of q and k at st->pos and the KV write (984-992).
hipError_t pi_launch_rope_kv(float *q, const float *k, const float *v, const float *cos_tab,
                             const float *sin_tab, const pi_state *st, float *kc_layer,
                             float *vc_layer, uint32_t n_head, uint32_t n_kv, uint32_t dh,
                             uint32_t half, uint32_t n_ctx, hipStream_t s);

// Single-token attention (model.rs:993-1087) in the reference's float order:
// scores in parallel over chunks of 64 positions (neon: f32_dot order at batch
// 1, else the scalar dot), then per head the serial softmax sum and value
// accumulation, fused with Q8 quantization of the output.  `scores` holds
// n_head * n_ctx floats.
hipError_t pi_launch_attention(const float *q, const float *kc_layer, const float *vc_layer,
                               const pi_state *st, uint32_t n_head, uint32_t n_kv, uint32_t dh,
                               uint32_t n_ctx, float scale, float *scores, uint32_t nchunk,
                               float *attn_out, int8_t *q8, float *d8, int32_t *s8, bool neon, hipStream_t s);

// Greedy argmax (sampler.rs:26-36): first index of the maximum.  Writes
// st->tok, ids[st->n_gen++], and advances st->pos.
hipError_t pi_launch_argmax(const float *logits, uint32_t n, float *pv, uint32_t *pidx,
                            pi_state *st, uint32_t *ids, hipStream_t s);
// Prefill advance: st->pos++, st->i++, st->tok = prompt[st->i].
hipError_t pi_launch_advance(pi_state *st, const uint32_t *prompt, hipStream_t s);

// Fills n positions of every (layer, kv head) with N(0,1) draws.
hipError_t pi_launch_kv_fill(float *kc, float *vc, uint32_t n_layer_heads, uint32_t n_ctx,
                             uint32_t dh, uint32_t n, uint64_t seed, hipStream_t s);

// Number of partial-argmax blocks used by pi_launch_argmax.
constexpr uint32_t PI_ARGMAX_BLOCKS = 256;
