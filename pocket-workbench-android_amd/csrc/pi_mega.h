// Persistent decode kernel: one cooperative launch evaluates one token
// through every layer (and, with the head, its greedy id).  Stages hand their
// outputs to each other through flag-tagged 64-bit words (value bits in the
// low half, the launch's epoch in the high half) written and read at device
// scope, so a consumer waits only for the words it needs: no grid barrier and
// no kernel boundary between stages.
#pragma once

#include <hip/hip_runtime_api.h>

#include "pi_gemv.h"

// Per-layer descriptor (a device-resident array, one entry per layer).
struct pi_mega_layer {
    pig::MatSet qkv;      // attn_q, attn_k (and attn_v when it shares their layout)
    pig::MatSet vb;       // attn_v when its type differs (vb.n == 0 otherwise)
    pig::MatSet o;        // attn_output
    pig::MatSet gu;       // ffn_gate, ffn_up (equal tile counts)
    pig::MatSet down;     // ffn_down
    uint32_t t_qkv, t_vb, t_o, g_o, t_gu, t_down, g_down;
    uint32_t h_q8;        // 1: h is published as Q8 blocks (pi_mega_h_blocks), else as floats
    const float *attn_norm, *ffn_norm;
    float *kc, *vc;       // this layer's [n_kv][n_ctx][head_dim] caches
    // flag-tagged words written during this layer
    uint64_t *q, *k, *v;  // projections (qdim, kdim, kdim words)
    uint64_t *att;        // Q8 of the attention output: qdim/4 quant words, qdim/32 scales, qdim/32 sums
    uint64_t *xb;         // residual after attn_output (n_embd words)
    uint64_t *h;          // SwiGLU output: n_ff float words, or with h_q8 n_ff/4 quant words, n_ff/32 scales, n_ff/32 sums
    uint64_t *xo;         // residual after ffn_down (n_embd words)
};

// Everything of a bound model the kernel reads; kept in device memory (the
// kernel receives a pointer) so no copy of it lands in scratch.
struct pi_mega_args {
    const pi_mega_layer *layers;
    uint32_t n_layer, ne, n_ff, n_head, n_kv, half, n_ctx, pad_;
    float eps, scale;
    const float *cos_tab, *sin_tab;
    const uint8_t *embd;      // token_embd rows in their native layout
    uint64_t erow_bytes;
    uint32_t etype, t_head;
    pig::MatSet head;         // output (logits y[0] unused: logits below)
    const float *out_norm;
    float *logits;
    uint64_t *part;           // 2 words per workgroup: argmax value bits, index
    uint32_t *tok_state;      // receives the greedy id (head launches)
    int32_t *abort_flag;      // set when a wait exceeds its spin bound
    uint64_t *trace;          // optional per-workgroup stage timestamps
    // Long-context attention (positions split into segments over several
    // workgroups); words tagged with epoch * 64 + layer + 1, shared by all layers:
    uint64_t *amax;           // per head, per segment: maximum score (n_head * PI_MEGA_MAX_SEG)
    uint64_t *aexp;           // per head, per position: e_p (n_head * n_ctx)
};

constexpr uint32_t PI_MEGA_MAX_SEG = 8;   // segments per head at most
constexpr uint32_t PI_MEGA_SEG_LEN = 1024;   // positions per segment at least (one segment below)

// What changes from launch to launch.
struct pi_mega_launch {
    const uint32_t *tok_src;  // token of this launch (null: tok_imm)
    uint32_t *id_out;         // also receives the greedy id when not null
    uint32_t tok_imm;
    int32_t pos;
    uint32_t epoch;           // tag of this launch's words (never 0)
};

// Flag-tagged words of one layer: q, k, v, att, xb, h, xo.
PI_HD inline uint64_t pi_mega_layer_words(uint32_t ne, uint32_t n_ff, uint32_t qdim, uint32_t kdim) {
    return (uint64_t)qdim + 2ull * kdim + (qdim / 4 + qdim / 16) + ne + n_ff + ne;
}
// Stage timestamps per workgroup when tracing: start, embedding, 5 per
// layer, head, then 32 points inside the stages of the middle layer.
PI_HD inline uint32_t pi_mega_trace_slots(uint32_t n_layer) { return 4 + 5 * n_layer + 32; }

size_t pi_mega_lds_bytes(uint32_t ne, uint32_t n_ff, uint32_t n_ctx);
// Whether the gate/up stage can run workgroups that each own whole Q8 blocks
// of h (32 rows of gate and of up, eight per wavefront) for gate/up tensors of
// this type and units per row: every lane holds at most three units of one
// column, and the four wavefronts' term strips fit the h staging area.
bool pi_mega_h_blocks(uint32_t type, uint32_t upr, uint32_t ne, uint32_t n_ff, uint32_t n_ctx);
// Workgroups the launch uses (one per CU when the kernel fits), 0 on error.
uint32_t pi_mega_blocks(int device, uint32_t ne, uint32_t n_ff, uint32_t n_ctx);
// neon: batch-1 float orders (else the multi-token chunk orders);
// head: output norm, head GEMV and greedy id after the layers.
// a: host copy (validated here); a_dev: the same bytes in device memory.
hipError_t pi_launch_mega(const pi_mega_args &a, const pi_mega_args *a_dev, const pi_mega_launch &l, bool neon,
                          bool head, uint32_t blocks, size_t lds, hipStream_t s);
