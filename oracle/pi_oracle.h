/*
 * pi_oracle.h -- CPU oracle for the pocketinfer decode path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  This is the checker: a plain-C
 * restatement of the reference engine's CPU path as built for aarch64 (its
 * only build with the int8 matmul), used only by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  The HIP library
 * never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference's rust/pocketinfer/src/).  Float expressions keep the
 * reference's evaluation order; the file is compiled with -ffp-contract=off
 * because Rust never contracts a*b+c into an FMA on its own.
 */
#ifndef PI_ORACLE_H
#define PI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (quant.rs:3-17). */
enum {
    PO_F32 = 0, PO_F16 = 1, PO_Q4_0 = 2, PO_Q4_1 = 3, PO_Q5_0 = 6, PO_Q5_1 = 7,
    PO_Q8_0 = 8, PO_Q8_1 = 9, PO_Q2_K = 10, PO_Q3_K = 11, PO_Q4_K = 12,
    PO_Q5_K = 13, PO_Q6_K = 14, PO_Q8_K = 15, PO_BF16 = 30
};

/* util.rs:76-100 / util.rs:102-138 */
float    po_f16_to_f32(uint16_t h);
uint16_t po_f32_to_f16(float v);

/* quant.rs:19-37: elements per block and bytes per block; 0 if unsupported. */
int po_type_block(uint32_t t, size_t *be, size_t *bb);
/* quant.rs:60-72: byte size of a tensor; returns 0 on success, -1 on error. */
int po_tensor_nbytes(uint32_t t, uint64_t ne0, uint64_t ne1, size_t *out);

/* ---- Q8 activations (quant_int.rs:3-56, simd_q8.rs:8-51) ---------------- */
/* x is feature-major/batch-minor: x[(blk*32+j)*b + bi].
 * Outputs are lane-major: q[bi*k + j], d[bi*nb + blk], sum[bi*nb + blk]. */
void po_q8_prepare(const float *x, size_t k, size_t b, int8_t *q, float *d, int32_t *sum);

typedef struct {
    const int8_t  *q;
    const float   *d;
    const int32_t *sum;
    size_t k, b, nb;
} po_q8act;

/* ---- int8 dots ----------------------------------------------------------- */
/* Single-lane forms dp::{q8_0,q4_0,q4_k,q6_k} (quant_int.rs:82-253). */
float po_dot_row_q8(uint32_t t, const uint8_t *row, size_t k, const po_q8act *act, size_t lane);
/* Multi-lane forms lanes::* (quant_int.rs:255-419); out[lane] += acc[lane]. */
void  po_dot_row_q8_lanes(uint32_t t, const uint8_t *row, size_t k, const po_q8act *act,
                          float *out, size_t b);
/* Integer sums of one row against one lane, in the reference's grouping:
 * per 32 elements for Q4_K/Q4_0/Q8_0, per 16 for Q6_K (quant_int.rs:330-419).
 * Returns the number of sums written, or -1 for an unsupported type. */
long  po_block_sums(uint32_t t, const uint8_t *row, size_t k, const po_q8act *act, size_t lane,
                    int32_t *sums);

/* ---- f32-activation path (quant.rs:102-476) ------------------------------ */
void  po_dequant_row(uint32_t t, const uint8_t *data, size_t k, float *out);
float po_dot_row_scalar(uint32_t t, const uint8_t *data, size_t k, const float *x);
void  po_row_dot_multi(uint32_t t, const uint8_t *row, size_t k, const float *xt, size_t b,
                       float *out);

/* ---- Pool (model.rs:139-350) --------------------------------------------- */
typedef struct po_pool po_pool;
po_pool *po_pool_new(int threads);
void     po_pool_free(po_pool *p);
/* Pool::matmul (model.rs:241-321): zero out[0..rows*b], then each row r
 * writes out[r*b .. r*b+b].  act == NULL selects the f32 path. */
void po_pool_matmul(po_pool *p, uint32_t t, const uint8_t *w, size_t row_bytes, size_t k,
                    const float *xt, size_t b, float *out, size_t rows, const po_q8act *act);

/* ---- Sampler (sampler.rs:1-92) ------------------------------------------- */
typedef struct { uint64_t s; } po_rng;
void     po_rng_init(po_rng *r, uint64_t seed);
uint64_t po_rng_next_u64(po_rng *r);
float    po_rng_next_f32(po_rng *r);
uint32_t po_sample(float *logits, size_t n, float temp, float top_p, po_rng *r);

/* ---- Model / engine (model.rs:14-1352) ----------------------------------- */
typedef struct {
    uint32_t type;
    size_t   ne0, ne1;          /* ne0 = row length (columns), ne1 = rows */
    const uint8_t *data;        /* row-major, row_bytes = tensor_nbytes(type, ne0) */
} po_tensor;

typedef struct {
    po_tensor attn_q, attn_k, attn_v, attn_o, attn_norm;
    po_tensor ffn_gate, ffn_up, ffn_down, ffn_norm;
} po_layer;

typedef struct {
    size_t n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_rot, n_vocab;
    float  rope_theta, rms_eps;
    const uint32_t *eos_ids;    /* Tokenizer::is_eog set (tokenizer.rs:252-254) */
    size_t n_eos;
    po_tensor token_embd, output, output_norm;
    const po_layer *layers;     /* n_layer entries */
} po_model;

typedef struct po_engine po_engine;

po_engine *po_engine_create(const po_model *m, size_t n_ctx, int threads, char *err, size_t errlen);
void       po_engine_destroy(po_engine *e);
void       po_engine_set_int8(po_engine *e, int enabled);
/* Engine::forward (model.rs:825-831): invalidates prefix reuse. 0 = ok. */
int        po_forward(po_engine *e, const uint32_t *ids, const size_t *pos, size_t b, int want_logits);
const float *po_logits(const po_engine *e);
size_t     po_n_logits(const po_engine *e);
float     *po_kv_k(po_engine *e);            /* KvCache::k (model.rs:352-359), pub */
float     *po_kv_v(po_engine *e);
size_t     po_kv_index(const po_engine *e, size_t l, size_t h, size_t pos, size_t d);
const char *po_last_error(const po_engine *e);

typedef struct {
    size_t   max_tokens;
    float    temp, top_p;
    uint64_t seed;
} po_genopts;

typedef struct {
    size_t prefill_tokens, prefill_cached_tokens, gen_tokens;
    double prefill_ms, gen_ms;
    char   stop[32];
} po_genstats;

/* Engine::generate (model.rs:1235-1352) without the text callback.
 * gen_ids must hold max_tokens entries.  0 = ok. */
int  po_generate(po_engine *e, const uint32_t *prompt, size_t n, const po_genopts *o,
                 po_genstats *st, uint32_t *gen_ids);

/* The deterministic exp / cos / sin / pow the oracle uses (po_detmath.h). */
float po_det_expf(float x);
float po_det_cosf(float x);
float po_det_sinf(float x);
float po_det_powf(float x, float y);

/* util.rs:274-282 */
void po_request_stop(void);
void po_clear_stop(void);

#ifdef __cplusplus
}
#endif
#endif
