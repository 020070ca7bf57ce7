/*
 * pocketinfer_hip.h -- C ABI of the MI355X (gfx950) decode backend for pocketinfer.
 *
 * Plain C: pointers, sizes and status codes only.  Every call returns 0 on
 * success or a negative PI_E_* code; the message of the last error of a
 * context is available from pi_last_error(ctx).  A context owns one HIP
 * stream, is used by one thread at a time (the reference backend is Send but
 * not Sync, backend/opencl.rs:94) and never falls back to a CPU path: on any
 * error it reports the error and leaves the fallback decision to the caller,
 * as Engine::matmul does (model.rs:736-743).
 *
 * Reference paths are relative to rust/pocketinfer/src/ of
 * Aleinto97/pocket-workbench-android.
 */
#ifndef POCKETINFER_HIP_H
#define POCKETINFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PI_ABI_VERSION 1

/* Status codes. */
#define PI_OK              0
#define PI_E_INVALID      -1   /* bad argument or shape */
#define PI_E_UNSUPPORTED  -2   /* tensor type without a HIP kernel */
#define PI_E_HIP          -3   /* HIP runtime error or no device */
#define PI_E_SELFTEST     -4   /* self-test mismatch against the CPU rule */
#define PI_E_NOMEM        -5   /* device or host allocation failed */
#define PI_E_INJECTED     -6   /* failure forced by pi_hip_fail_next */
#define PI_E_STOPPED      -7   /* cooperative stop (util.rs:274-282) */
#define PI_E_CONTEXT_FULL -8   /* position >= n_ctx (model.rs:847-850) */
#define PI_E_NOMODEL      -9   /* whole-forward call before pi_hip_model_bind */

/* GGML tensor type ids (quant.rs:3-17). */
#define PI_TYPE_F32  0u
#define PI_TYPE_F16  1u
#define PI_TYPE_Q4_0 2u
#define PI_TYPE_Q4_1 3u
#define PI_TYPE_Q5_0 6u
#define PI_TYPE_Q5_1 7u
#define PI_TYPE_Q8_0 8u
#define PI_TYPE_Q8_1 9u
#define PI_TYPE_Q2_K 10u
#define PI_TYPE_Q3_K 11u
#define PI_TYPE_Q4_K 12u
#define PI_TYPE_Q5_K 13u
#define PI_TYPE_Q6_K 14u
#define PI_TYPE_Q8_K 15u
#define PI_TYPE_BF16 30u

typedef struct pi_ctx pi_ctx;
typedef struct pi_tensor pi_tensor;   /* weights resident in HBM */

/* ---------------------------------------------------------------------------
 * Backend twin of OpenClBackend (backend/opencl.rs).
 * ------------------------------------------------------------------------- */

/* probe() (opencl.rs:235-258): writes a NUL-terminated device description
 * into buf and returns 0 when a gfx950 device is visible; PI_E_HIP otherwise. */
int         pi_hip_probe(char *buf, size_t n);
/* OpenClBackend::new (opencl.rs:260-379): device index, own stream. */
int         pi_hip_create(pi_ctx **out, int device);
/* Drop for OpenClBackend (opencl.rs:503-516): frees weights, buffers, stream. */
void        pi_hip_destroy(pi_ctx *ctx);
/* OpenClBackend::name (opencl.rs:381-383). */
const char *pi_hip_name(const pi_ctx *ctx);
/* util::Error message of the last failed call on ctx (util.rs:5-43). */
const char *pi_last_error(const pi_ctx *ctx);
/* OpenClBackend::supports (opencl.rs:432-434): 1 for the int8-path types
 * Q4_K, Q6_K, Q4_0, Q8_0 (quant_int.rs:75-80: Q8 of x, then the lanes
 * epilogue), and for Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K and BF16,
 * which the reference evaluates on its f32 path (quant::dot_row,
 * quant.rs:361-441: products of dequantized weights and f32 x added in
 * element order).  Q2_K, Q3_K and Q5_K follow the GGUF layout; the
 * reference's decoders of those three index past their slices and panic
 * (quant.rs:211, 254, 295-314). */
int         pi_hip_supports(const pi_ctx *ctx, uint32_t ggml_type);
/* OpenClBackend::selftest (opencl.rs:391-430): the same Q4_K and Q6_K vectors
 * and tolerance |gpu-cpu| <= 0.02|cpu| + 0.01, with cpu the f32 dot_row. */
int         pi_hip_selftest(pi_ctx *ctx);
/* OpenClBackend::matvec (opencl.rs:436-500): out[rows] = W[rows x k] x.
 * Host pointers.  w is uploaded once per (w, w_bytes) and kept in HBM
 * (opencl.rs:439-460); x is quantized to Q8 blocks on the device. */
int         pi_hip_matvec(pi_ctx *ctx, uint32_t ggml_type, const uint8_t *w, size_t w_bytes,
                          size_t k, const float *x, float *out, size_t rows);
/* OpenClBackend::clear_weight_cache (opencl.rs:385-389). */
void        pi_hip_clear_weight_cache(pi_ctx *ctx);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, hosts that
 * forbid hipMalloc): out[rows] = W x for a tensor already uploaded with
 * pi_hip_upload, x (k floats) and out (rows floats) in host memory, with the
 * same results as pi_hip_matvec.  It allocates nothing: x and y are staged
 * in a static device array of (PI_NOALLOC_MAX_K + PI_NOALLOC_MAX_ROWS) * 4
 * bytes per GPU, held until the process ends; larger tensors are rejected
 * with PI_E_INVALID.  Every call on one GPU shares that array, so calls that
 * overlap on one GPU (from several contexts or threads) race.  Synchronous. */
#define PI_NOALLOC_MAX_K    16384u
#define PI_NOALLOC_MAX_ROWS 262144u
int         pi_hip_matvec_noalloc(pi_ctx *ctx, const pi_tensor *w, const float *x, float *out);

/* ---------------------------------------------------------------------------
 * Explicit upload and device-pointer GEMV (no counterpart call in the
 * reference; it replaces the implicit upload inside matvec, opencl.rs:439-460).
 * Weights of the int8-path types are repacked on the device into a tiled
 * layout: each row is cut into units of whole blocks, one unit per lane of a
 * 64-wide wavefront tile, and the 16-byte chunks of the units are interleaved
 * across the lanes so a wavefront reads one contiguous span per load; f16
 * block scales of Q6_K, Q4_0 and Q8_0 move to a plane of their own.  The
 * native bytes are not kept.  The f32-path types keep their GGUF rows.
 * ------------------------------------------------------------------------- */
int  pi_hip_upload(pi_ctx *ctx, uint32_t ggml_type, const void *host, size_t rows, size_t k,
                   pi_tensor **out);
void pi_hip_tensor_free(pi_ctx *ctx, pi_tensor *t);
/* Bytes the tensor occupies in HBM (the algorithmic weight bytes). */
size_t pi_hip_tensor_bytes(const pi_tensor *t);
/* y[rows] = W x with x and y device pointers, on the context stream.
 * Int8-path types, one launch: every workgroup quantizes x (k floats) to Q8
 * blocks in its LDS (quant_int.rs:17-56), then runs the fused dequant +
 * int8-dot GEMV (quant_int.rs:330-419).  (Rows too long for LDS take a Q8
 * pre-pass into context staging memory instead; same results.)  f32-path
 * types: each row's dequantized weights times x are added in element order
 * (quant.rs:377-441) by one lane per row while other wavefronts form the
 * products. */
int  pi_hip_gemv_dev(pi_ctx *ctx, const pi_tensor *w, const float *x_dev, float *y_dev);
/* Same GEMV on already-quantized activations (device pointers, lane 0);
 * int8-path types only (PI_E_UNSUPPORTED otherwise). */
int  pi_hip_gemv_q8_dev(pi_ctx *ctx, const pi_tensor *w, const int8_t *q_dev, const float *d_dev,
                        const int32_t *sum_dev, float *y_dev);
/* Times `iters` launches of the GEMV kernel alone on the context stream with
 * HIP events; writes the mean kernel time in microseconds.  When n_copies > 1,
 * launch i uses weights[i % n_copies] so the timed reads come from HBM rather
 * than the 256 MB Infinity Cache. */
int  pi_hip_time_gemv(pi_ctx *ctx, const pi_tensor *const *weights, int n_copies, const int8_t *q_dev,
                      const float *d_dev, const int32_t *sum_dev, float *y_dev, int iters,
                      double *avg_us);

/* Times `iters` runs of the whole pi_hip_gemv_dev job (Q8 of the f32 x in
 * HBM, then the GEMV) with HIP events on the context stream; writes the mean
 * time per run in microseconds.  Weight copies rotate as in pi_hip_time_gemv.
 * No counterpart in the reference (its matvec times nothing, opencl.rs:436-500). */
int  pi_hip_time_gemv_x(pi_ctx *ctx, const pi_tensor *const *weights, int n_copies, const float *x_dev,
                        float *y_dev, int iters, double *avg_us);

/* Q8Act::prepare on device buffers (x feature-major [k][b]), context stream. */
int  pi_hip_q8_quantize_dev(pi_ctx *ctx, const float *x_dev, size_t k, int b, int8_t *q_dev, float *d_dev,
                            int32_t *sum_dev);

/* Device memory for callers without an allocator of their own (a Rust host,
 * tests, benchmarks): hipMalloc / hipFree / synchronous copies on the
 * context's device. */
int  pi_hip_dev_alloc(pi_ctx *ctx, size_t bytes, void **out);
void pi_hip_dev_free(pi_ctx *ctx, void *p);
int  pi_hip_copy_h2d(pi_ctx *ctx, void *dst_dev, const void *src, size_t bytes);
int  pi_hip_copy_d2h(pi_ctx *ctx, void *dst, const void *src_dev, size_t bytes);
/* Device-to-device copy on the context stream (asynchronous): a streaming
 * copy kernel for the 16-byte-aligned bulk, so HBM counters can be calibrated
 * against a copy of known size. */
int  pi_hip_copy_d2d(pi_ctx *ctx, void *dst_dev, const void *src_dev, size_t bytes);

/* Stream control.  pi_hip_set_stream makes the context launch on a caller
 * stream (a hipStream_t passed as a plain pointer; NULL restores its own). */
int  pi_hip_set_stream(pi_ctx *ctx, void *hip_stream);
int  pi_hip_synchronize(pi_ctx *ctx);

/* ---------------------------------------------------------------------------
 * Test hooks for the bit-exact contract.
 * ------------------------------------------------------------------------- */
/* Q8Act::prepare (quant_int.rs:17-56) on the device.  Host pointers.
 * x is feature-major/batch-minor x[(blk*32+j)*b + bi]; outputs are
 * lane-major q[bi*k+j], d[bi*(k/32)+blk], sum[bi*(k/32)+blk]. */
int  pi_hip_q8_quantize(pi_ctx *ctx, const float *x, size_t k, int b, int8_t *q, float *d,
                        int32_t *sum);
/* Integer block sums of every row of w against lane 0 of a Q8 activation
 * (host pointers): per 32 elements for Q4_K/Q4_0/Q8_0, per 16 for Q6_K in
 * the visiting order of quant_int.rs:397-413.  sums holds rows*k/32 (or
 * rows*k/16 for Q6_K) entries, row-major. */
int  pi_hip_block_sums(pi_ctx *ctx, const pi_tensor *w, const int8_t *q, const float *d,
                       const int32_t *sum, int32_t *sums);
/* Makes the next matvec / gemv / forward on ctx fail with PI_E_INJECTED, so
 * callers can exercise their CPU fallback (model.rs:736-743). */
int  pi_hip_fail_next(pi_ctx *ctx);

/* ---------------------------------------------------------------------------
 * Whole-forward engine: the device-resident counterpart of Engine
 * (model.rs:678-1352).  Weights are uploaded once; the KV cache, scratch,
 * RoPE tables and logits live in HBM.
 * ------------------------------------------------------------------------- */
typedef struct {
    uint32_t    type;         /* ggml type id */
    uint64_t    ne0, ne1;     /* columns (row length), rows */
    const void *data;         /* host bytes, e.g. an mmap'd GGUF tensor */
} pi_tensor_desc;

typedef struct {              /* LayerWeights (model.rs:474-484) */
    pi_tensor_desc attn_q, attn_k, attn_v, attn_o, attn_norm;
    pi_tensor_desc ffn_gate, ffn_up, ffn_down, ffn_norm;
} pi_layer_desc;

typedef struct {              /* Config (model.rs:14-29) + tensors */
    uint32_t n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_rot, n_vocab;
    float    rope_theta, rms_eps;
    const uint32_t *eos_ids;  /* Tokenizer::is_eog set (tokenizer.rs:252-254) */
    uint32_t n_eos;
    pi_tensor_desc token_embd, output, output_norm;
    const pi_layer_desc *layers;
} pi_model_desc;

typedef struct {              /* GenOpts (model.rs:657-664): temp <= 0 is greedy */
    uint32_t max_tokens;
    float    temp, top_p;
    uint64_t seed;
} pi_genopts;

typedef struct {              /* GenStats (model.rs:666-676) */
    uint32_t prefill_tokens, prefill_cached_tokens, gen_tokens;
    double   prefill_ms, gen_ms;
    char     stop[32];        /* "max_tokens" | "eog" | "user_stop" | "context_full" */
} pi_genstats;

/* Engine::load (model.rs:698-723) + Model::finish shape checks (571-601):
 * uploads every tensor, allocates an f32 KV cache of n_ctx positions. */
int  pi_hip_model_bind(pi_ctx *ctx, const pi_model_desc *m, uint32_t n_ctx);
/* Engine::forward (model.rs:825-831): evaluates b tokens (1 <= b <= 64) at the
 * given positions, writes their K/V rows, and when want_logits computes the
 * logits of the last token.  Invalidates prefix reuse, as the reference does. */
int  pi_hip_forward(pi_ctx *ctx, const uint32_t *ids, const int32_t *pos, int b, int want_logits);
/* Engine::logits (model.rs:1231-1233): copies n <= n_vocab logits to host. */
int  pi_hip_logits(pi_ctx *ctx, float *out, size_t n);
/* Greedy sample (sampler.rs:26-36) on the device: first index of the max. */
int  pi_hip_argmax(pi_ctx *ctx, uint32_t *id);
/* Engine::generate (model.rs:1235-1352): 32-token prefill chunks with the
 * reference reuse rule (1258-1268), n tokens for n-1 forwards, is_eog stop.
 * temp <= 0 is greedy and stays on the device; temp > 0 draws each token with
 * sample() (sampler.rs:21-92, seeded with opts->seed) on the host from the
 * logits of the last forward, and leaves the last draw's weights in the
 * logits, as the reference's sample() does. */
int  pi_hip_generate(pi_ctx *ctx, const uint32_t *prompt, size_t n, const pi_genopts *opts,
                     pi_genstats *stats, uint32_t *gen_ids);
/* Direct KV access (KvCache is pub, model.rs:352-359): rows for positions
 * pos0..pos0+n of one layer and kv head, [n][head_dim] f32, host pointers. */
int  pi_hip_kv_write(pi_ctx *ctx, uint32_t layer, uint32_t kv_head, uint32_t pos0, uint32_t n,
                     const float *k, const float *v);
int  pi_hip_kv_read(pi_ctx *ctx, uint32_t layer, uint32_t kv_head, uint32_t pos0, uint32_t n,
                    float *k, float *v);
/* Fills the KV rows of positions [0, n) of every layer and head with
 * N(0,1) draws of a seeded generator, on the device (long-context setup);
 * pi_synth_kv_normal gives the same values on the host. */
int  pi_hip_kv_fill_normal(pi_ctx *ctx, uint32_t n, uint64_t seed);
/* Marks positions [0, n) of the KV cache as holding these tokens, so that
 * forward/generate may continue from them (used after pi_hip_kv_write). */
int  pi_hip_kv_set_tokens(pi_ctx *ctx, const uint32_t *ids, uint32_t n);
/* util::request_stop / STOP_REQUESTED reset (util.rs:274-282), per context. */
void pi_hip_request_stop(pi_ctx *ctx);
void pi_hip_clear_stop(pi_ctx *ctx);
/* Engine steps replay captured HIP graphs by default; enable = 0 launches the
 * same kernels one by one (for profilers that cannot follow graph launches). */
int  pi_hip_use_graphs(pi_ctx *ctx, int enable);
/* Engine tokens run as one persistent cooperative kernel per token by default
 * (stages hand data to each other through flag-tagged words in HBM); enable
 * = 0 selects the per-stage kernels instead.  No counterpart in the
 * reference: the reference evaluates a token as a sequence of CPU loops. */
int  pi_hip_use_persistent(pi_ctx *ctx, int enable);
/* Prompt chunks of 2..32 tokens (and engine forwards of several consecutive
 * tokens) run on the batched int8-MFMA prefill kernels by default, in passes
 * that may span several chunks; enable = 0 evaluates them one token at a
 * time.  Results are identical either way (the reference's multi-token float
 * orders, model.rs:812-822, 1028-1038). */
int  pi_hip_use_batch_prefill(pi_ctx *ctx, int enable);
/* Tokens per batched prefill pass of the bound model: 1024, halved while the
 * pass's attention scores (pass * n_head * n_ctx floats) exceed 1 GiB; 0 when
 * no model is bound or it is outside the batched kernels' limits.  No
 * counterpart in the reference, whose passes are its 32-token chunks. */
int  pi_hip_prefill_pass_tokens(const pi_ctx *ctx);
/* 1 when the bound model runs on the persistent kernel, 0 otherwise. */
int  pi_hip_persistent_active(const pi_ctx *ctx);
/* Stage tracing of the persistent kernel (the reference's GenStats wall
 * times, model.rs:666-676, at stage granularity): when enabled, every
 * workgroup records the 100 MHz device clock at the end of each stage of the
 * last launch.  pi_hip_stage_trace_read copies blocks*slots entries
 * (workgroup-major: start, embedding, 5 per layer, head); out = NULL only
 * reports blocks and slots. */
int  pi_hip_stage_trace(pi_ctx *ctx, int enable);
int  pi_hip_stage_trace_read(pi_ctx *ctx, uint64_t *out, size_t n, uint32_t *blocks, uint32_t *slots);
/* Per-forward timing of the last generate call, microseconds (device events
 * around the whole decode loop, host waits included). */
int  pi_hip_last_decode_us(pi_ctx *ctx, double *per_token_us);
/* Kernel timing of generate (the reference's GenStats timing, model.rs:666-676,
 * at kernel granularity): when enabled, every decode forward is bracketed by
 * an event pair, and pi_hip_last_kernel_us reports the mean device time of
 * one forward's kernels over the n forwards of the last generate call. */
int  pi_hip_time_kernels(pi_ctx *ctx, int enable);
int  pi_hip_last_kernel_us(pi_ctx *ctx, double *per_forward_us, uint32_t *n);

/* ---------------------------------------------------------------------------
 * GGUF reader (gguf.rs), host-side.  The file is mapped read-only; tensor
 * data and the model descriptor point into the mapping, which stays valid
 * until pi_gguf_close.  Errors copy a message into err (err_len bytes).
 * ------------------------------------------------------------------------- */
typedef struct pi_gguf pi_gguf;
/* Gguf::load (gguf.rs:113-192): MappedFile::open (util.rs:163-192) + parse
 * of a GGUF v2/v3 header, metadata and tensor table. */
int         pi_gguf_open(const char *path, pi_gguf **out, char *err, size_t err_len);
/* Gguf::parse over bytes the caller keeps alive (no copy). */
int         pi_gguf_parse(const void *bytes, size_t len, pi_gguf **out, char *err, size_t err_len);
void        pi_gguf_close(pi_gguf *g);
uint32_t    pi_gguf_version(const pi_gguf *g);
/* Gguf::data_offset: start of the tensor data (aligned to general.alignment). */
uint64_t    pi_gguf_data_offset(const pi_gguf *g);
/* Gguf::keys (gguf.rs:198-200): metadata keys in file order. */
size_t      pi_gguf_n_kv(const pi_gguf *g);
const char *pi_gguf_key(const pi_gguf *g, size_t i);
/* The GGUF value type of a key (0 U8 ... 12 F64). */
int         pi_gguf_kv_type(const pi_gguf *g, const char *key, uint32_t *type);
/* Gguf::get_u64 / get_f32 / get_bool / get_str (gguf.rs:206-255). */
int         pi_gguf_get_u64(const pi_gguf *g, const char *key, uint64_t *v);
int         pi_gguf_get_f32(const pi_gguf *g, const char *key, float *v);
int         pi_gguf_get_bool(const pi_gguf *g, const char *key, int *v);
int         pi_gguf_get_str(const pi_gguf *g, const char *key, const char **s, size_t *len);
/* Gguf::array_len / array_type / array_strings / array_i32 / array_f32
 * (gguf.rs:257-316). */
int         pi_gguf_array_info(const pi_gguf *g, const char *key, uint32_t *etype, uint64_t *count);
int         pi_gguf_array_str(const pi_gguf *g, const char *key, uint64_t i, const char **s, size_t *len);
int         pi_gguf_array_i32(const pi_gguf *g, const char *key, int32_t *out, size_t n);
int         pi_gguf_array_f32(const pi_gguf *g, const char *key, float *out, size_t n);
/* Gguf::tensors / tensor / tensor_data (gguf.rs:318-336). */
size_t      pi_gguf_n_tensors(const pi_gguf *g);
int64_t     pi_gguf_find_tensor(const pi_gguf *g, const char *name);
int         pi_gguf_tensor_info(const pi_gguf *g, size_t i, const char **name, uint32_t *type, uint32_t *n_dims,
                                uint64_t ne[4], uint64_t *offset);
int         pi_gguf_tensor_data(const pi_gguf *g, size_t i, const void **data, size_t *nbytes, char *err,
                                size_t err_len);
/* Config::from_gguf (model.rs:31-97) and Model::load's tensor binding and
 * shape checks (model.rs:487-601), with the tokenizer's vocabulary size and
 * end-of-generation ids (tokenizer.rs:41-109): fills *m for
 * pi_hip_model_bind.  layers holds max_layers entries, eos max_eos ids. */
int         pi_gguf_model_desc(const pi_gguf *g, pi_model_desc *m, pi_layer_desc *layers, uint32_t max_layers,
                               uint32_t *eos, uint32_t max_eos, char *err, size_t err_len);

/* ---------------------------------------------------------------------------
 * Sampling (sampler.rs), host-side.
 * ------------------------------------------------------------------------- */
/* Rng::new (sampler.rs:6-8): the SplitMix64 state for a seed. */
uint64_t pi_rng_new(uint64_t seed);
/* Rng::next_u64 (sampler.rs:9-15): advances *state. */
uint64_t pi_rng_next_u64(uint64_t *state);
/* sample (sampler.rs:21-92): greedy for temp <= 0, else temperature and
 * top-p over n logits (overwritten with the weights, as the reference's
 * &mut [f32] is), drawing from *rng_state.  Equal weights are ordered by
 * index in the top-p cut (the reference's sort_unstable_by leaves them in an
 * unspecified order). */
uint32_t pi_sample(float *logits, size_t n, float temp, float top_p, uint64_t *rng_state);

/* ---------------------------------------------------------------------------
 * Seeded synthetic data (host-side, deterministic across machines: integer
 * SplitMix64 (sampler.rs:1-19) and IEEE double arithmetic only).
 * ------------------------------------------------------------------------- */
/* Random Q4_K blocks: d, dmin ~ U[dlo, dhi] as f16; 12 scale bytes and 128
 * quant bytes uniform. */
int pi_synth_q4k_random(uint64_t seed, size_t rows, size_t k, float dlo, float dhi, uint8_t *out);
/* Random Q6_K blocks: ql/qh uniform bytes; scales uniform in [-64, 63];
 * d ~ U[dlo, dhi] as f16. */
int pi_synth_q6k_random(uint64_t seed, size_t rows, size_t k, float dlo, float dhi, uint8_t *out);
/* The values pi_hip_kv_fill_normal writes for positions p0..p0+n-1 of
 * layer-major kv head lh (= layer * n_kv + head): k and v get n * dh floats,
 * [position][dim].  Host-only, bit-identical to the device fill. */
int pi_synth_kv_normal(uint64_t seed, uint32_t lh, uint32_t p0, uint32_t n, uint32_t dh, float *k, float *v);
/* n draws of N(mean, std) (Marsaglia polar method). */
int pi_synth_normal(uint64_t seed, size_t n, float mean, float std, float *out);
/* rows x k weights ~ N(mean, std), quantized row by row to ggml_type (F32
 * copies them).  Row r draws from its own stream, so the bytes do not depend
 * on `threads`. */
int pi_synth_tensor(uint64_t seed, uint32_t ggml_type, size_t rows, size_t k, float mean, float std,
                    uint8_t *out, int threads);
/* Quantizes one row of k floats to ggml_type blocks (a plain amax/min-max
 * encoder; the reference ships no quantizer, make_tiny_model.py:5). */
int pi_quantize_row(uint32_t ggml_type, const float *x, size_t k, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
