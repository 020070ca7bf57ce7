// Launchers of the batched prefill kernels (pi_prefill.hip): one pass of up
// to PI_PF_MAX_TOK consecutive prompt tokens evaluated together, in the float
// orders the reference uses for a batch of more than one token (model.rs:
// 812-822, 1028-1038).  A token's values depend only on its own inputs and on
// the KV rows of earlier positions, so a pass may span several of the
// reference's 32-token chunks without changing any value.
// All launch on `s` and return hipSuccess or the launch error.
#pragma once

#include <hip/hip_runtime_api.h>

#include "pi_common.h"

constexpr uint32_t PI_PF_MAX_TOK = 1024;
// Score scratch a pass may use (pi_pf_attn): the engine halves its pass size
// from PI_PF_MAX_TOK until the pass's scores fit.
constexpr uint64_t PI_PF_SCORE_BUDGET = 1ull << 30;

// A weight matrix in the tiled layout (pi_common.h), as the prefill GEMM reads it.
struct pi_pf_mat {
    const uint8_t *w;
    pi_layout L;
};

// Token-major activations of a chunk: row t of a [ntok][n] matrix at t * n.
// Q8 activations (the values of Q8Act, quant_int.rs:17-56) are laid out for
// the MFMA operand loads: the 8 quants 8*ka..8*ka+7 of 32-element group G of
// token t at byte ((G * 4 + ka) * PI_PF_MAX_TOK + t) * 8; d and the block sum
// of (G, t) at index G * PI_PF_MAX_TOK + t.
struct pi_pf_q8 {
    int8_t *q;
    float *d;
    int32_t *s;
};

// X[t] = token_embd row ids[t] (dequant_row, model.rs:857-869).
hipError_t pi_pf_embed(const uint8_t *embd, uint32_t etype, uint64_t row_bytes, const uint32_t *ids_dev, uint32_t ntok,
                       uint32_t ne, float *X, hipStream_t s);
// RMSNorm of every token in the scalar order (model.rs:812-822), then Q8.
hipError_t pi_pf_norm_q8(const float *X, const float *w, uint32_t ne, float eps, uint32_t ntok, pi_pf_q8 out,
                         hipStream_t s);
// out[t][row] = W a_t (resid: out[t][row] += W a_t); int8 MFMA for the integer
// sums of every 32- (Q6_K: 16-) element group, the reference's float
// epilogue in block order per (row, token).
hipError_t pi_pf_gemm(const pi_pf_mat &W, pi_pf_q8 act, uint32_t ntok, float *out, bool resid, hipStream_t s);
// What the GEMM does with an output of 64-dimension heads (rows a multiple
// of 64) instead of storing it: RoPE of its pairs (model.rs:953-979) into a
// token-major matrix (Q), RoPE then the rows of positions pos0..pos0+ntok-1
// of a [head][n_ctx][64] cache (K, 984-992), or the cache rows alone (V).
enum pi_pf_out : uint32_t { PI_PF_STORE = 0, PI_PF_ROPE = 1, PI_PF_ROPE_CACHE = 2, PI_PF_CACHE = 3 };
struct pi_pf_rope {
    const float *cos_tab, *sin_tab;   // [n_ctx][half]
    uint32_t pos0, half, n_ctx;
};
// The same for up to 3 matrices of one type and row length sharing the
// activation, in one launch; out[i] is a [ntok][rows of M[i]] matrix, or the
// layer's cache for the cache modes (mode = nullptr: all PI_PF_STORE; the
// other modes need rope and resid == false).
hipError_t pi_pf_gemm_multi(const pi_pf_mat *M, float *const *out, const uint32_t *mode, uint32_t nseg, pi_pf_q8 act,
                            uint32_t ntok, bool resid, const pi_pf_rope *rope, hipStream_t s);
// Attention of every token over positions 0..its own (model.rs:993-1087,
// multi-token orders), then Q8 of the output.  scores: scratch of
// ntok * n_head * pi_pf_score_stride(n_ctx) floats.
constexpr uint64_t pi_pf_score_stride(uint32_t n_ctx) { return ((uint64_t)n_ctx + 31) & ~31ull; }
hipError_t pi_pf_attn(const float *Q, const float *kc, const float *vc, uint32_t pos0, uint32_t ntok, uint32_t n_head,
                      uint32_t n_kv, uint32_t n_ctx, float scale, float *scores, pi_pf_q8 out, hipStream_t s);
// h = silu(gate) * up (model.rs:1111-1115), then Q8 of h.
hipError_t pi_pf_swiglu_q8(const float *G, const float *U, uint32_t ntok, uint32_t n_ff, pi_pf_q8 out, hipStream_t s);
