// Launchers of the fused decode kernels (pi_decode.hip) and of the
// standalone GEMV.  All launch on `s`, return hipSuccess or the launch error,
// and never synchronize.
#pragma once

#include <hip/hip_runtime_api.h>

#include "pi_kernels.h"

// Up to three matrices of one type and layout that share an activation;
// tiles are numbered back to back, tile0[m] being the first tile of matrix m
// and tile0[n] the total.
struct pi_matset {
    const uint8_t *w[3];
    float *y[3];
    uint32_t rows[3];
    uint32_t tile0[4];
    uint32_t n;
    pi_layout L;   // common layout (rows of the first matrix)
};

enum pi_epi { PI_EPI_OUT = 0, PI_EPI_SWIGLU = 1, PI_EPI_ARGMAX = 2 };
enum pi_pro { PI_PRO_GLOBAL = 0, PI_PRO_Q8 = 1 };
enum pi_step_mode { PI_STEP_ARGMAX = 0, PI_STEP_PROMPT = 1, PI_STEP_EMBED = 2 };

// RMSNorm of x (ne floats, weight nw) + Q8, then the GEMVs of A and B (B may
// be empty; A and B then have 256-element units).  epi: OUT writes y;
// SWIGLU needs A = {gate, up} and writes h = silu(gate)*up; ARGMAX writes y
// and one (max, index) pair per workgroup into pv/pidx.
struct pi_norm_gemv_args {
    const float *x, *nw;
    uint32_t ne;
    float eps;
    pi_matset A, B;
    float *h;
    float *pv;
    uint32_t *pidx;
    int epi;
    uint32_t blocks;
};

// GEMV with x[row] += value on a Q8 activation in HBM (pro = GLOBAL: aq, ad,
// as) or quantized in the kernel from the f32 vector hx of k floats (pro =
// Q8).
struct pi_gemv_res_args {
    const int8_t *aq;
    const float *ad;
    const int32_t *as;
    const float *hx;
    uint32_t k;
    pi_matset M;
    int pro;
    uint32_t blocks;
};

// Single-token attention of all heads for the token at st->pos.
struct pi_attn_args {
    const float *q, *k, *v;
    const float *cos_tab, *sin_tab;
    const pi_state *st;
    float *kc, *vc;   // this layer's [n_kv][n_ctx][dh] caches
    uint32_t n_head, n_kv, dh, n_ctx, half;
    float scale;
    int8_t *oq;
    float *od;
    int32_t *os;
};

// Standalone GEMV over a matrix set (mode OUT / RESIDUAL / SUMS; SUMS needs
// n == 1): `blocks` persistent wavefronts, four per workgroup.
hipError_t pi_launch_gemv_set(const pi_matset &M, const int8_t *aq, const float *ad, const int32_t *as,
                              int32_t *sums, int mode, uint32_t blocks, hipStream_t s);
// Standalone GEMV on an f32 x (k floats in HBM): each workgroup quantizes x
// to Q8 blocks in its LDS, then runs the tiles (mode OUT).
hipError_t pi_launch_gemv_x(const pi_matset &M, const float *x, uint32_t blocks, hipStream_t s);
// LDS bytes of that kernel for a layout (type, units of g blocks, row length k).
size_t pi_gemv_x_lds_bytes(uint32_t type, uint32_t g, uint32_t k);
hipError_t pi_launch_norm_gemv(const pi_norm_gemv_args &a, bool neon, hipStream_t s);
hipError_t pi_launch_gemv_res(const pi_gemv_res_args &a, hipStream_t s);
hipError_t pi_launch_attn(const pi_attn_args &a, bool neon, hipStream_t s);
size_t pi_attn_lds_bytes(uint32_t n_ctx);
// mode ARGMAX: greedy id from np partials -> st->tok, ids[st->n_gen++],
// st->pos++; PROMPT: st->pos++, st->i++, st->tok = prompt[st->i]; EMBED: no
// state change.  Then x = embedding row of st->tok.
hipError_t pi_launch_step(int mode, const float *pv, const uint32_t *pidx, uint32_t np, pi_state *st,
                          uint32_t *ids, const uint32_t *prompt, const uint8_t *embd, uint32_t etype, uint32_t ne,
                          uint64_t row_bytes, float *x, hipStream_t s);
