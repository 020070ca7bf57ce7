// C ABI of the pocketinfer MI355X backend: the OpenClBackend twin
// (backend/opencl.rs), explicit upload, test hooks and the device-resident
// engine (model.rs:678-1352).  Host code only; kernels are in pi_kernels.hip.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "pi_common.h"
#include "pi_detmath.h"
#include "pi_decode.h"
#include "pi_kernels.h"
#include "pi_mega.h"
#include "pi_prefill.h"
#include "pi_rowdot.h"
#include "pi_sample.h"

struct pi_tensor {
    pi_layout L;
    uint8_t *dev = nullptr;
};

// Staging memory of pi_hip_matvec_noalloc: x (PI_NOALLOC_MAX_K floats), then
// y (PI_NOALLOC_MAX_ROWS floats).  One copy per GPU, held until the process
// ends.  In host code `scratch` only names the symbol: kernels and copies use
// the device address hipGetSymbolAddress returns for each device.
constexpr size_t kScratchBytes = ((size_t)PI_NOALLOC_MAX_K + PI_NOALLOC_MAX_ROWS) * 4;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};
bool g_scratch_done[kMaxDevices] = {};

// Device address of this device's `scratch`, looked up once per device with
// that device current (pi_hip_create); null when the lookup failed.
void *scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_done[device]) {
        void *p = nullptr;
        g_scratch_err[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[device] = g_scratch_err[device] == hipSuccess ? p : nullptr;
        g_scratch_done[device] = true;
    }
    return g_scratch_ptr[device];
}
}  // namespace

namespace {

// Persistent grid cap of the standalone GEMV, in wavefronts (4 per workgroup):
// 1024 = one workgroup on each of the 256 CUs.  Measured on the 122753x2304
// Q6_K head: 40.4 us at 1024 against 44-45 us at 2048, 47 at 1536, 49 at 768;
// a grid that puts a second workgroup on some CUs leaves the others idle at the end.
constexpr uint32_t kGemvMaxBlocks = 1024;
constexpr uint32_t kFusedMaxBlocks = 1024; // persistent grid cap of the fused kernels (4 waves each)
constexpr uint32_t kMaxBatch = 64;     // model.rs:12
constexpr uint32_t kDecodeChunk = 16;  // decode steps launched between host checks

struct Layer {
    pi_tensor *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    pi_tensor *gate = nullptr, *up = nullptr, *down = nullptr;
    float *attn_norm = nullptr, *ffn_norm = nullptr;
};

struct Engine {
    uint32_t n_layer = 0, n_embd = 0, n_ff = 0, n_head = 0, n_kv = 0, dh = 0, n_rot = 0, n_vocab = 0;
    float eps = 1e-5f, theta = 10000.f;
    uint32_t n_ctx = 0;
    std::vector<uint32_t> eos;
    std::vector<Layer> layers;
    uint8_t *embd = nullptr;
    uint32_t embd_type = 0;
    uint64_t embd_row_bytes = 0;
    pi_tensor *head = nullptr;
    float *out_norm = nullptr;
    float *kc = nullptr, *vc = nullptr, *cos_tab = nullptr, *sin_tab = nullptr;
    float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *h = nullptr, *logits = nullptr,
          *amax_v = nullptr;
    uint32_t *amax_i = nullptr, *ids = nullptr, *prompt = nullptr;
    int8_t *q8q = nullptr;    // Q8 of the attention output (input of attn_o)
    float *q8d = nullptr;
    int32_t *q8s = nullptr;
    pi_state *st = nullptr;
    // graphs: layers in the batch-1 (NEON) and batch>1 (scalar) orders, logits,
    // decode step, prefill step, and the last prompt token of a multi-token chunk
    hipGraphExec_t g_layers_neon = nullptr, g_layers_seq = nullptr, g_logits = nullptr, g_decode = nullptr,
                   g_prefill = nullptr, g_last_seq = nullptr;
    std::vector<uint32_t> kv_tokens;
    size_t cached_prefill_len = 0;
    double last_decode_us = 0.0;
    double last_kernel_us = 0.0;    // mean device time of one decode forward's kernels (kernel timing on)
    uint32_t last_kernel_n = 0;
    // persistent decode kernel (pi_mega.hip)
    bool mega_ok = false;           // the model fits the kernel
    pi_mega_args mega{};            // host copy of the device-resident arguments
    pi_mega_args *mega_dev = nullptr;
    pi_mega_layer *mega_layers = nullptr;
    uint64_t *mega_words = nullptr; // flag-tagged hand-off words of every layer
    uint64_t *mega_part = nullptr;
    int32_t *mega_abort = nullptr;
    uint64_t *mega_trace = nullptr;  // per-workgroup stage timestamps when tracing
    uint64_t *mega_amax = nullptr, *mega_aexp = nullptr;   // long-context attention words
    uint32_t mega_blocks = 0, epoch = 0;
    size_t mega_lds = 0;
    // batched prefill (pi_prefill.hip): token-major chunk buffers
    bool pf_ok = false;
    uint32_t pf_pass = 0;   // tokens per device pass (a multiple of 64, at most PI_PF_MAX_TOK)
    float *pfX = nullptr, *pfQ = nullptr, *pfG = nullptr, *pfU = nullptr;
    float *pfS = nullptr;   // attention scores of a pass: [token][head][n_ctx]
    int8_t *pfq = nullptr;
    float *pfd = nullptr;
    int32_t *pfs = nullptr;
    uint32_t *pf_ids = nullptr;
};

}  // namespace

struct pi_ctx {
    int device = 0;
    hipStream_t own = nullptr, stream = nullptr;
    std::string name, err;
    bool fail_next = false;
    bool use_graphs = true;   // replay captured graphs (else launch each kernel)
    bool use_persistent = true;  // one persistent kernel per token when the model fits
    bool use_batch_prefill = true;  // multi-token chunks on the MFMA prefill kernels
    bool time_kernels = false;      // event pair around every decode forward of generate
    std::atomic<int> stop{0};
    std::map<std::pair<uintptr_t, size_t>, pi_tensor *> wcache;
    // grow-only IO buffers of matvec / test hooks (opencl.rs:461-482)
    float *io_x = nullptr, *io_y = nullptr;
    int8_t *io_q = nullptr;
    float *io_d = nullptr;
    int32_t *io_s = nullptr;
    size_t cap_x = 0, cap_y = 0;
    int max_lds = 65536;      // LDS bytes a workgroup may use on this device
    void *scratch = nullptr;  // this device's `scratch` (pi_hip_matvec_noalloc)
    Engine *eng = nullptr;
};

namespace {

int fail(pi_ctx *c, int code, const char *fmt, ...) {
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return code;
}

#define HIPC(c, expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess) return fail((c), PI_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

bool take_injected(pi_ctx *c) {
    if (!c->fail_next) return false;
    c->fail_next = false;
    c->err = "injected failure";
    return true;
}

template <typename T>
int dalloc(pi_ctx *c, T **p, size_t n) {
    *p = nullptr;
    if (n == 0) n = 1;
    hipError_t e = hipMalloc((void **)p, n * sizeof(T));
    if (e != hipSuccess) return fail(c, PI_E_NOMEM, "hipMalloc(%zu bytes): %s", n * sizeof(T), hipGetErrorString(e));
    return PI_OK;
}

void dfree(void *p) {
    if (p) (void)hipFree(p);
}

int grow_io(pi_ctx *c, size_t k, size_t rows) {
    if (k > c->cap_x) {
        dfree(c->io_x); dfree(c->io_q); dfree(c->io_d); dfree(c->io_s);
        c->io_x = nullptr; c->io_q = nullptr; c->io_d = nullptr; c->io_s = nullptr;
        c->cap_x = 0;
        int r;
        if ((r = dalloc(c, &c->io_x, k)) || (r = dalloc(c, &c->io_q, k)) || (r = dalloc(c, &c->io_d, k / 32 + 1)) ||
            (r = dalloc(c, &c->io_s, k / 32 + 1)))
            return r;
        c->cap_x = k;
    }
    if (rows > c->cap_y) {
        dfree(c->io_y);
        c->io_y = nullptr;
        c->cap_y = 0;
        int r = dalloc(c, &c->io_y, rows);
        if (r) return r;
        c->cap_y = rows;
    }
    return PI_OK;
}

// Upload native rows (host) and repack on the device.
int upload_tensor(pi_ctx *c, uint32_t type, const void *host, size_t rows, size_t k, pi_tensor **out) {
    *out = nullptr;
    if (!pi_gemv_type(type) && !pi_row_type(type)) return fail(c, PI_E_UNSUPPORTED, "tensor type %u has no HIP kernel", type);
    if (!host || rows == 0 || rows > 0xFFFFFFFFu || k == 0 || k > 0xFFFFFFFFu)
        return fail(c, PI_E_INVALID, "invalid upload arguments");
    if (pi_row_type(type)) {
        // f32-path types keep their GGUF rows (BF16 rows of a multiple of 32)
        const size_t rb = pi_row_bytes(type, k);
        if (rb == 0 || k % 32 || pi_gemv_row_lds_bytes((uint32_t)k) > (size_t)c->max_lds)
            return fail(c, PI_E_INVALID, "row length %zu not supported for type %u", k, type);
        pi_tensor *t = new pi_tensor();
        t->L = pi_layout{};
        t->L.type = type;
        t->L.k = (uint32_t)k;
        t->L.rows = (uint32_t)rows;
        t->L.bytes = (uint64_t)rb * rows;
        int r = dalloc(c, &t->dev, t->L.bytes);
        if (r) { delete t; return r; }
        hipError_t e = hipMemcpyAsync(t->dev, host, t->L.bytes, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            dfree(t->dev);
            delete t;
            return fail(c, PI_E_HIP, "upload: %s", hipGetErrorString(e));
        }
        *out = t;
        return PI_OK;
    }
    pi_layout L;
    if (!pi_make_layout(type, (uint32_t)rows, (uint32_t)k, &L))
        return fail(c, PI_E_INVALID, "row length %zu not supported for type %u", k, type);
    size_t nbytes = pi_row_bytes(type, k) * rows;
    uint8_t *staging = nullptr;
    int r = dalloc(c, &staging, nbytes);
    if (r) return r;
    pi_tensor *t = new pi_tensor();
    t->L = L;
    r = dalloc(c, &t->dev, L.bytes);
    if (r) { dfree(staging); delete t; return r; }
    hipError_t e = hipMemcpyAsync(staging, host, nbytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(t->dev, 0, L.bytes, c->stream);
    if (e == hipSuccess) e = pi_launch_repack(staging, t->dev, L, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    dfree(staging);
    if (e != hipSuccess) {
        dfree(t->dev);
        delete t;
        return fail(c, PI_E_HIP, "upload: %s", hipGetErrorString(e));
    }
    *out = t;
    return PI_OK;
}

void free_tensor(pi_tensor *t) {
    if (!t) return;
    dfree(t->dev);
    delete t;
}

// The self-test comparator: quant::dot_row as the reference evaluates it on
// x86 for the two test blocks (quant.rs:377-441).  It only checks the GPU; it
// is never used to produce results.
float selftest_dot_q4k(const uint8_t *b, const float *x) {
    float d = pi_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))), dmin = pi_f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
    const uint8_t *sc = b + 4, *qs = b + 16;
    float tmp[256];
    for (int is = 0; is < 8; is += 2) {
        uint32_t s[2], m[2];
        for (int t = 0; t < 2; t++) {
            int j = is + t;
            if (j < 4) { s[t] = sc[j] & 63u; m[t] = sc[j + 4] & 63u; }
            else { s[t] = (sc[j + 4] & 0xFu) | ((sc[j - 4] >> 6) << 4); m[t] = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4); }
        }
        float d1 = d * (float)s[0], m1 = dmin * (float)m[0], d2 = d * (float)s[1], m2 = dmin * (float)m[1];
        for (int l = 0; l < 32; l++) tmp[is * 32 + l] = d1 * (float)(qs[is / 2 * 32 + l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) tmp[is * 32 + 32 + l] = d2 * (float)(qs[is / 2 * 32 + l] >> 4) - m2;
    }
    float sum = 0.0f;
    for (int j = 0; j < 256; j++) sum += tmp[j] * x[j];
    return sum;
}

float selftest_dot_q6k(const uint8_t *b, const float *x) {
    float d = pi_f16_to_f32((uint16_t)(b[208] | (b[209] << 8))), acc = 0.0f;
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    for (int half = 0; half < 2; half++)
        for (int l = 0; l < 32; l++) {
            int is = l / 16, qlb = half * 64, qhb = half * 32, o = half * 128;
            int q1 = (int)((ql[qlb + l] & 0xF) | (((qh[qhb + l] >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql[qlb + l + 32] & 0xF) | (((qh[qhb + l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[qlb + l] >> 4) | (((qh[qhb + l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[qlb + l + 32] >> 4) | (((qh[qhb + l] >> 6) & 3) << 4)) - 32;
            acc += d * (float)sc[half * 8 + is] * (float)q1 * x[o + l];
            acc += d * (float)sc[half * 8 + is + 2] * (float)q2 * x[o + 32 + l];
            acc += d * (float)sc[half * 8 + is + 4] * (float)q3 * x[o + 64 + l];
            acc += d * (float)sc[half * 8 + is + 6] * (float)q4 * x[o + 96 + l];
        }
    return acc;
}

// ---------------------------------------------------------------------------
// Engine
// ---------------------------------------------------------------------------
void engine_free(Engine *e) {
    if (!e) return;
    for (hipGraphExec_t g : {e->g_layers_neon, e->g_layers_seq, e->g_logits, e->g_decode, e->g_prefill, e->g_last_seq})
        if (g) (void)hipGraphExecDestroy(g);
    for (Layer &l : e->layers) {
        for (pi_tensor *t : {l.q, l.k, l.v, l.o, l.gate, l.up, l.down}) free_tensor(t);
        dfree(l.attn_norm);
        dfree(l.ffn_norm);
    }
    free_tensor(e->head);
    for (void *p : {(void *)e->mega_dev, (void *)e->mega_layers, (void *)e->mega_words, (void *)e->mega_part,
                    (void *)e->mega_abort, (void *)e->mega_trace, (void *)e->mega_amax, (void *)e->mega_aexp})
        dfree(p);
    for (void *p : {(void *)e->pfX, (void *)e->pfQ, (void *)e->pfG, (void *)e->pfU,
                    (void *)e->pfS, (void *)e->pfq, (void *)e->pfd, (void *)e->pfs, (void *)e->pf_ids})
        dfree(p);
    for (void *p : {(void *)e->embd, (void *)e->out_norm, (void *)e->kc, (void *)e->vc, (void *)e->cos_tab,
                    (void *)e->sin_tab, (void *)e->x, (void *)e->q, (void *)e->k, (void *)e->v, (void *)e->h,
                    (void *)e->logits, (void *)e->amax_v, (void *)e->amax_i, (void *)e->ids, (void *)e->prompt,
                    (void *)e->q8q, (void *)e->q8d, (void *)e->q8s, (void *)e->st})
        dfree(p);
    delete e;
}

bool check_shape(const pi_tensor_desc &t, uint64_t cols, uint64_t rows) { return t.ne0 == cols && t.ne1 == rows; }

int upload_norm(pi_ctx *c, const pi_tensor_desc &t, uint32_t ne, float **out) {
    if (t.type != PI_TYPE_F32) return fail(c, PI_E_UNSUPPORTED, "norm weights must be F32 (type %u)", t.type);
    int r = dalloc(c, out, ne);
    if (r) return r;
    HIPC(c, hipMemcpy(*out, t.data, (size_t)ne * 4, hipMemcpyHostToDevice));
    return PI_OK;
}

int upload_mat(pi_ctx *c, const pi_tensor_desc &t, pi_tensor **out) {
    return upload_tensor(c, t.type, t.data, (size_t)t.ne1, (size_t)t.ne0, out);
}

// Matrix set over tensors of one type and layout (tiles back to back).
pi_matset make_set(std::initializer_list<std::pair<const pi_tensor *, float *>> mats) {
    pi_matset S{};
    uint32_t t = 0, i = 0;
    for (const auto &m : mats) {
        S.w[i] = m.first->dev;
        S.y[i] = m.second;
        S.rows[i] = m.first->L.rows;
        S.tile0[i] = t;
        t += m.first->L.ntiles;
        i++;
    }
    S.n = i;
    for (uint32_t j = i; j < 4; j++) S.tile0[j] = t;
    if (i) S.L = mats.begin()->first->L;
    return S;
}

bool same_layout(const pi_tensor *a, const pi_tensor *b) {
    return a->L.type == b->L.type && a->L.k == b->L.k && a->L.g == b->L.g;
}

uint32_t fused_blocks(uint32_t tiles) {
    uint32_t b = (tiles + 3) / 4;
    return b < 1 ? 1 : (b > kFusedMaxBlocks ? kFusedMaxBlocks : b);
}

uint32_t gemv_blocks(uint32_t tiles) { return tiles < kGemvMaxBlocks ? (tiles ? tiles : 1) : kGemvMaxBlocks; }

hipError_t launch_single_gemv(const pi_tensor *w, const int8_t *q, const float *d, const int32_t *s, float *y,
                              int32_t *sums, int mode, hipStream_t st) {
    const pi_matset M = make_set({{w, y}});
    return pi_launch_gemv_set(M, q, d, s, sums, mode, gemv_blocks(w->L.ntiles), st);
}

// Enqueues the layers of one token whose embedding is in x; st holds pos.
hipError_t enqueue_layers(const Engine &e, bool neon, hipStream_t s) {
    hipError_t r;
#define K(expr) do { if ((r = (expr)) != hipSuccess) return r; } while (0)
    const float scale = 1.0f / sqrtf((float)e.dh);
    for (uint32_t l = 0; l < e.n_layer; l++) {
        const Layer &L = e.layers[l];
        float *kc = e.kc + (uint64_t)l * e.n_kv * e.n_ctx * e.dh;
        float *vc = e.vc + (uint64_t)l * e.n_kv * e.n_ctx * e.dh;
        // attn_norm + Q/K/V
        pi_norm_gemv_args a{};
        a.x = e.x; a.nw = L.attn_norm; a.ne = e.n_embd; a.eps = e.eps; a.epi = PI_EPI_OUT;
        if (same_layout(L.q, L.k) && same_layout(L.q, L.v)) {
            a.A = make_set({{L.q, e.q}, {L.k, e.k}, {L.v, e.v}});
        } else if (same_layout(L.q, L.k)) {
            a.A = make_set({{L.q, e.q}, {L.k, e.k}});
            a.B = make_set({{L.v, e.v}});
        } else {
            return hipErrorInvalidValue;  // bind rejects this combination
        }
        a.blocks = fused_blocks(a.A.tile0[3] + a.B.tile0[3]);
        K(pi_launch_norm_gemv(a, neon, s));
        // RoPE + KV write + attention + Q8 of the output
        pi_attn_args t{};
        t.q = e.q; t.k = e.k; t.v = e.v; t.cos_tab = e.cos_tab; t.sin_tab = e.sin_tab; t.st = e.st;
        t.kc = kc; t.vc = vc; t.n_head = e.n_head; t.n_kv = e.n_kv; t.dh = e.dh; t.n_ctx = e.n_ctx;
        t.half = e.n_rot / 2; t.scale = scale; t.oq = e.q8q; t.od = e.q8d; t.os = e.q8s;
        K(pi_launch_attn(t, neon, s));
        // attn_o + residual
        pi_gemv_res_args o{};
        o.aq = e.q8q; o.ad = e.q8d; o.as = e.q8s; o.k = e.n_embd; o.pro = PI_PRO_GLOBAL;
        o.M = make_set({{L.o, e.x}});
        o.blocks = fused_blocks(o.M.tile0[3]);
        K(pi_launch_gemv_res(o, s));
        // ffn_norm + gate/up + SwiGLU
        pi_norm_gemv_args f{};
        f.x = e.x; f.nw = L.ffn_norm; f.ne = e.n_embd; f.eps = e.eps; f.epi = PI_EPI_SWIGLU; f.h = e.h;
        f.A = make_set({{L.gate, e.h}, {L.up, e.h}});
        f.blocks = fused_blocks(L.gate->L.ntiles);
        K(pi_launch_norm_gemv(f, neon, s));
        // Q8 of h + ffn_down + residual
        pi_gemv_res_args d{};
        d.hx = e.h; d.k = e.n_ff; d.pro = PI_PRO_Q8;
        d.M = make_set({{L.down, e.x}});
        d.blocks = fused_blocks(d.M.tile0[3]);
        K(pi_launch_gemv_res(d, s));
    }
    return hipSuccess;
}

// output_norm + head GEMV (the head always normalizes one column: the batch-1
// order, model.rs:1136-1143) with per-workgroup argmax partials.
hipError_t enqueue_logits(const Engine &e, hipStream_t s) {
    pi_norm_gemv_args a{};
    a.x = e.x; a.nw = e.out_norm; a.ne = e.n_embd; a.eps = e.eps; a.epi = PI_EPI_ARGMAX;
    a.A = make_set({{e.head, e.logits}});
    a.pv = e.amax_v; a.pidx = e.amax_i;
    a.blocks = PI_HEAD_BLOCKS;
    return pi_launch_norm_gemv(a, true, s);
}

// mode: PI_STEP_ARGMAX (greedy id of the last logits), PI_STEP_PROMPT (next
// prompt token) or PI_STEP_EMBED; then the embedding of st->tok goes to x.
hipError_t enqueue_step(const Engine &e, int mode, uint32_t *ids, hipStream_t s) {
    return pi_launch_step(mode, e.amax_v, e.amax_i, PI_HEAD_BLOCKS, e.st, ids, e.prompt, e.embd, e.embd_type,
                          e.n_embd, e.embd_row_bytes, e.x, s);
}
#undef K

template <typename F>
hipError_t capture(hipStream_t s, hipGraphExec_t *out, F enqueue) {
    hipGraph_t g = nullptr;
    hipError_t r = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (r != hipSuccess) return r;
    hipError_t er = enqueue();
    r = hipStreamEndCapture(s, &g);
    if (er != hipSuccess) { if (g) (void)hipGraphDestroy(g); return er; }
    if (r != hipSuccess) return r;
    r = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    return r;
}

int build_graphs(pi_ctx *c, Engine &e) {
    hipStream_t s = c->stream;
    HIPC(c, capture(s, &e.g_layers_neon, [&] { return enqueue_layers(e, true, s); }));
    HIPC(c, capture(s, &e.g_layers_seq, [&] { return enqueue_layers(e, false, s); }));
    HIPC(c, capture(s, &e.g_logits, [&] { return enqueue_logits(e, s); }));
    for (int neon = 0; neon < 2; neon++)
        HIPC(c, capture(s, neon ? &e.g_decode : &e.g_last_seq, [&] {
            hipError_t r = enqueue_layers(e, neon != 0, s);
            if (r == hipSuccess) r = enqueue_logits(e, s);
            if (r == hipSuccess) r = enqueue_step(e, PI_STEP_ARGMAX, e.ids, s);
            return r;
        }));
    HIPC(c, capture(s, &e.g_prefill, [&] {
        hipError_t r = enqueue_layers(e, false, s);
        if (r == hipSuccess) r = enqueue_step(e, PI_STEP_PROMPT, nullptr, s);
        return r;
    }));
    return PI_OK;
}

// Kernel-side view of tensors of one layout, tiles numbered back to back.
pig::MatSet mset(std::initializer_list<const pi_tensor *> ts) {
    pig::MatSet S{};
    uint32_t t = 0, i = 0;
    for (const pi_tensor *x : ts) {
        S.w[i] = x->dev;
        S.y[i] = nullptr;
        S.rows[i] = x->L.rows;
        S.tile0[i] = t;
        t += x->L.ntiles;
        i++;
    }
    S.n = i;
    for (uint32_t j = i; j < 4; j++) S.tile0[j] = t;
    if (i) {
        const pi_layout &L = (*ts.begin())->L;
        S.upr = L.upr;
        S.rpw = L.rpw;
        S.lpt = L.lpt;
        S.tile_bytes = L.tile_bytes;
    }
    return S;
}

// Sets up the persistent decode kernel for a bound model; leaves mega_ok
// false (per-stage kernels are used) when the model is outside its limits.
int build_mega(pi_ctx *c, Engine &e) {
    e.mega_ok = false;
    const uint32_t qdim = e.n_head * e.dh, kdim = e.n_kv * e.dh;
    if (e.n_embd % 128 || e.n_ff % 128 || (e.n_head * e.dh) % 128 || e.n_embd / 16 > 256 || e.n_ff / 32 > 256 ||
        e.n_rot / 2 > 32 || e.dh != 64 || e.n_layer > 63)
        return PI_OK;
    int maxlds = 0;
    if (hipDeviceGetAttribute(&maxlds, hipDeviceAttributeSharedMemPerBlockOptin, c->device) != hipSuccess) maxlds = 65536;
    e.mega_lds = pi_mega_lds_bytes(e.n_embd, e.n_ff, e.n_ctx);
    if (e.mega_lds > (size_t)maxlds) return PI_OK;
    e.mega_blocks = pi_mega_blocks(c->device, e.n_embd, e.n_ff, e.n_ctx);
    if (e.mega_blocks < 2 * e.n_head) return PI_OK;   // two attention workgroups per head
    const uint64_t per = pi_mega_layer_words(e.n_embd, e.n_ff, qdim, kdim);
    int r;
    if ((r = dalloc(c, &e.mega_words, per * e.n_layer)) || (r = dalloc(c, &e.mega_part, 2ull * e.mega_blocks)) ||
        (r = dalloc(c, &e.mega_abort, 1)) || (r = dalloc(c, &e.mega_layers, e.n_layer)) || (r = dalloc(c, &e.mega_dev, 1)) ||
        (r = dalloc(c, &e.mega_amax, (uint64_t)e.n_head * PI_MEGA_MAX_SEG)) ||
        (r = dalloc(c, &e.mega_aexp, (uint64_t)e.n_head * e.n_ctx)))
        return r;
    HIPC(c, hipMemset(e.mega_amax, 0, (uint64_t)e.n_head * PI_MEGA_MAX_SEG * 8));
    HIPC(c, hipMemset(e.mega_aexp, 0, (uint64_t)e.n_head * e.n_ctx * 8));
    HIPC(c, hipMemset(e.mega_words, 0, per * e.n_layer * 8));
    HIPC(c, hipMemset(e.mega_part, 0, 2ull * e.mega_blocks * 8));
    HIPC(c, hipMemset(e.mega_abort, 0, 4));
    std::vector<pi_mega_layer> ly(e.n_layer);
    for (uint32_t l = 0; l < e.n_layer; l++) {
        const Layer &L = e.layers[l];
        pi_mega_layer &Y = ly[l];
        memset(&Y, 0, sizeof Y);
        if (same_layout(L.q, L.k) && same_layout(L.q, L.v)) {
            Y.qkv = mset({L.q, L.k, L.v});
        } else {
            Y.qkv = mset({L.q, L.k});
            Y.vb = mset({L.v});
        }
        Y.t_qkv = L.q->L.type;
        Y.t_vb = L.v->L.type;
        Y.o = mset({L.o});
        Y.t_o = L.o->L.type;
        Y.g_o = L.o->L.g;
        Y.gu = mset({L.gate, L.up});
        Y.t_gu = L.gate->L.type;
        Y.h_q8 = same_layout(L.gate, L.up) &&
                 pi_mega_h_blocks(L.gate->L.type, L.gate->L.upr, e.n_embd, e.n_ff, e.n_ctx);
        Y.down = mset({L.down});
        Y.t_down = L.down->L.type;
        Y.g_down = L.down->L.g;
        Y.attn_norm = L.attn_norm;
        Y.ffn_norm = L.ffn_norm;
        Y.kc = e.kc + (uint64_t)l * e.n_kv * e.n_ctx * e.dh;
        Y.vc = e.vc + (uint64_t)l * e.n_kv * e.n_ctx * e.dh;
        uint64_t *w = e.mega_words + per * l;
        Y.q = w; w += qdim;
        Y.k = w; w += kdim;
        Y.v = w; w += kdim;
        Y.att = w; w += qdim / 4 + qdim / 16;
        Y.xb = w; w += e.n_embd;
        Y.h = w; w += e.n_ff;
        Y.xo = w;
    }
    HIPC(c, hipMemcpy(e.mega_layers, ly.data(), ly.size() * sizeof(pi_mega_layer), hipMemcpyHostToDevice));
    pi_mega_args &a = e.mega;
    memset(&a, 0, sizeof a);
    a.layers = e.mega_layers;
    a.n_layer = e.n_layer; a.ne = e.n_embd; a.n_ff = e.n_ff; a.n_head = e.n_head; a.n_kv = e.n_kv;
    a.half = e.n_rot / 2; a.n_ctx = e.n_ctx;
    a.eps = e.eps; a.scale = 1.0f / sqrtf((float)e.dh);
    a.cos_tab = e.cos_tab; a.sin_tab = e.sin_tab;
    a.embd = e.embd; a.erow_bytes = e.embd_row_bytes; a.etype = e.embd_type;
    a.head = mset({e.head});
    a.t_head = e.head->L.type;
    a.out_norm = e.out_norm;
    a.logits = e.logits;
    a.part = e.mega_part;
    a.tok_state = &e.st->tok;
    a.abort_flag = e.mega_abort;
    a.trace = nullptr;
    a.amax = e.mega_amax;
    a.aexp = e.mega_aexp;
    HIPC(c, hipMemcpy(e.mega_dev, &a, sizeof a, hipMemcpyHostToDevice));
    e.mega_ok = true;
    return PI_OK;
}

bool use_mega(const pi_ctx *c, const Engine &e) { return c->use_persistent && e.mega_ok; }

// Buffers of the batched prefill; leaves pf_ok false (tokens are evaluated
// one by one) when the model is outside the kernels' limits.
int build_prefill(pi_ctx *c, Engine &e) {
    e.pf_ok = false;
    const uint32_t qdim = e.n_head * e.dh;
    if (e.dh != 64 || e.n_embd / 32 > 256 || e.n_rot / 2 > 32) return PI_OK;
    // Larger passes fill the machine better (the attention's workgroups come in
    // whole rounds, the weights stream once per pass); the attention scores of
    // a pass, pass * n_head * n_ctx floats, bound it at long context.
    const uint64_t srow = e.n_head * pi_pf_score_stride(e.n_ctx) * 4;
    uint32_t pass = PI_PF_MAX_TOK;
    while (pass > 64 && pass * srow > PI_PF_SCORE_BUDGET) pass /= 2;
    const uint64_t T = pass, TQ = PI_PF_MAX_TOK;   // Q8 activations keep the PI_PF_MAX_TOK stride
    const uint64_t kmax = std::max(std::max(e.n_embd, e.n_ff), qdim);
    int r;
    if ((r = dalloc(c, &e.pfX, T * e.n_embd)) || (r = dalloc(c, &e.pfQ, T * qdim)) ||
        (r = dalloc(c, &e.pfG, T * e.n_ff)) || (r = dalloc(c, &e.pfU, T * e.n_ff)) ||
        (r = dalloc(c, &e.pfq, TQ * kmax)) || (r = dalloc(c, &e.pfd, TQ * kmax / 32)) ||
        (r = dalloc(c, &e.pfs, TQ * kmax / 32)) || (r = dalloc(c, &e.pfS, T * e.n_head * pi_pf_score_stride(e.n_ctx))) ||
        (r = dalloc(c, &e.pf_ids, 2 * T)))
        return r;
    e.pf_pass = pass;
    e.pf_ok = true;
    return PI_OK;
}

bool use_pf(const pi_ctx *c, const Engine &e) { return c->use_batch_prefill && e.pf_ok; }

pi_pf_mat pfmat(const pi_tensor *t) { return pi_pf_mat{t->dev, t->L}; }

// One pass of ntok (1..pf_pass) consecutive tokens at positions pos0..
// through every layer on the batched prefill kernels; the residual stream
// ends in pfX.
hipError_t pf_chunk(const pi_ctx *c, const Engine &e, const uint32_t *ids_dev, uint32_t pos0, uint32_t ntok) {
    hipStream_t s = c->stream;
    hipError_t r;
#define K(expr) do { if ((r = (expr)) != hipSuccess) return r; } while (0)
    const float scale = 1.0f / sqrtf((float)e.dh);
    const pi_pf_q8 A{e.pfq, e.pfd, e.pfs};
    K(pi_pf_embed(e.embd, e.embd_type, e.embd_row_bytes, ids_dev, ntok, e.n_embd, e.pfX, s));
    for (uint32_t l = 0; l < e.n_layer; l++) {
        const Layer &L = e.layers[l];
        float *kc = e.kc + (uint64_t)l * e.n_kv * e.n_ctx * e.dh;
        float *vc = e.vc + (uint64_t)l * e.n_kv * e.n_ctx * e.dh;
        K(pi_pf_norm_q8(e.pfX, L.attn_norm, e.n_embd, e.eps, ntok, A, s));
        {
            // Q, K, V with RoPE and the cache rows of positions pos0.. formed
            // in the GEMM's epilogue (matrices of one type share a launch)
            const pi_pf_rope rp{e.cos_tab, e.sin_tab, pos0, e.n_rot / 2, e.n_ctx};
            const pi_pf_mat m[3] = {pfmat(L.q), pfmat(L.k), pfmat(L.v)};
            float *const o[3] = {e.pfQ, kc, vc};
            const uint32_t md[3] = {PI_PF_ROPE, PI_PF_ROPE_CACHE, PI_PF_CACHE};
            bool done[3] = {false, false, false};
            for (uint32_t i = 0; i < 3; i++) {
                if (done[i]) continue;
                pi_pf_mat gm[3];
                float *go[3];
                uint32_t gmd[3], n = 0;
                for (uint32_t j = i; j < 3; j++) {
                    if (done[j] || m[j].L.type != m[i].L.type || m[j].L.k != m[i].L.k) continue;
                    gm[n] = m[j];
                    go[n] = o[j];
                    gmd[n++] = md[j];
                    done[j] = true;
                }
                K(pi_pf_gemm_multi(gm, go, gmd, n, A, ntok, false, &rp, s));
            }
        }
        K(pi_pf_attn(e.pfQ, kc, vc, pos0, ntok, e.n_head, e.n_kv, e.n_ctx, scale, e.pfS, A, s));
        K(pi_pf_gemm(pfmat(L.o), A, ntok, e.pfX, true, s));
        K(pi_pf_norm_q8(e.pfX, L.ffn_norm, e.n_embd, e.eps, ntok, A, s));
        {
            const pi_pf_mat m[2] = {pfmat(L.gate), pfmat(L.up)};
            float *const o[2] = {e.pfG, e.pfU};
            if (m[1].L.type == m[0].L.type) {
                K(pi_pf_gemm_multi(m, o, nullptr, 2, A, ntok, false, nullptr, s));
            } else {
                K(pi_pf_gemm(m[0], A, ntok, e.pfG, false, s));
                K(pi_pf_gemm(m[1], A, ntok, e.pfU, false, s));
            }
        }
        K(pi_pf_swiglu_q8(e.pfG, e.pfU, ntok, e.n_ff, A, s));
        K(pi_pf_gemm(pfmat(L.down), A, ntok, e.pfX, true, s));
    }
    return hipSuccess;
#undef K
}

// One token through the persistent kernel (layers, and the head when `head`).
hipError_t mega_token(const pi_ctx *c, Engine &e, int32_t pos, uint32_t tok_imm, const uint32_t *tok_src,
                      uint32_t *id_out, bool neon, bool head) {
    // Epochs run 1 .. 2^26 - 1 (attention words carry epoch * 64 + layer + 1):
    // at the wrap every tagged word is cleared, so no stale word can carry the
    // tag a later launch waits for.
    if (++e.epoch >= (1u << 26)) {
        e.epoch = 1;
        const uint32_t qdim = e.n_head * e.dh, kdim = e.n_kv * e.dh;
        hipError_t r;
        if ((r = hipMemsetAsync(e.mega_words, 0, pi_mega_layer_words(e.n_embd, e.n_ff, qdim, kdim) * e.n_layer * 8,
                                c->stream)) != hipSuccess ||
            (r = hipMemsetAsync(e.mega_part, 0, 2ull * e.mega_blocks * 8, c->stream)) != hipSuccess ||
            (r = hipMemsetAsync(e.mega_amax, 0, (uint64_t)e.n_head * PI_MEGA_MAX_SEG * 8, c->stream)) != hipSuccess ||
            (r = hipMemsetAsync(e.mega_aexp, 0, (uint64_t)e.n_head * e.n_ctx * 8, c->stream)) != hipSuccess)
            return r;
    }
    pi_mega_launch l{tok_src, id_out, tok_imm, pos, e.epoch};
    return pi_launch_mega(e.mega, e.mega_dev, l, neon, head, e.mega_blocks, e.mega_lds, c->stream);
}

// Reads and clears the abort flag after the stream has drained.
int mega_check(pi_ctx *c, Engine &e) {
    if (!use_mega(c, e)) return PI_OK;
    int32_t f = 0;
    HIPC(c, hipMemcpy(&f, e.mega_abort, 4, hipMemcpyDeviceToHost));
    if (f) {
        HIPC(c, hipMemset(e.mega_abort, 0, 4));
        return fail(c, PI_E_HIP, "persistent decode kernel: a hand-off wait exceeded its bound");
    }
    return PI_OK;
}

enum StepKind { STEP_LAYERS_NEON, STEP_LAYERS_SEQ, STEP_LOGITS, STEP_DECODE, STEP_PREFILL, STEP_LAST_SEQ };

// One engine step on the context stream: a graph replay, or the same kernels
// launched one by one when graphs are off (for tools that cannot follow
// graph launches).
hipError_t run_step(const pi_ctx *c, const Engine &e, StepKind k) {
    hipStream_t s = c->stream;
    if (c->use_graphs) {
        const hipGraphExec_t g[] = {e.g_layers_neon, e.g_layers_seq, e.g_logits, e.g_decode, e.g_prefill, e.g_last_seq};
        return hipGraphLaunch(g[k], s);
    }
    hipError_t r = hipSuccess;
    switch (k) {
    case STEP_LAYERS_NEON: return enqueue_layers(e, true, s);
    case STEP_LAYERS_SEQ: return enqueue_layers(e, false, s);
    case STEP_LOGITS: return enqueue_logits(e, s);
    case STEP_PREFILL:
        r = enqueue_layers(e, false, s);
        return r == hipSuccess ? enqueue_step(e, PI_STEP_PROMPT, nullptr, s) : r;
    case STEP_DECODE:
    case STEP_LAST_SEQ:
        r = enqueue_layers(e, k == STEP_DECODE, s);
        if (r == hipSuccess) r = enqueue_logits(e, s);
        return r == hipSuccess ? enqueue_step(e, PI_STEP_ARGMAX, e.ids, s) : r;
    }
    return hipErrorInvalidValue;
}

int set_state(pi_ctx *c, Engine &e, int32_t pos, uint32_t tok, uint32_t n_gen, uint32_t i) {
    pi_state h{pos, tok, n_gen, i};
    HIPC(c, hipMemcpyAsync(e.st, &h, sizeof h, hipMemcpyHostToDevice, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

int pi_hip_probe(char *buf, size_t n) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        if (buf && n) snprintf(buf, n, "no HIP device");
        return PI_E_HIP;
    }
    for (int i = 0; i < count; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) != hipSuccess) continue;
        if (strncmp(p.gcnArchName, "gfx950", 6) == 0) {
            if (buf && n) snprintf(buf, n, "%s (%s, %d CUs, %.0f GiB)", p.name, p.gcnArchName, p.multiProcessorCount,
                                   (double)p.totalGlobalMem / (1024.0 * 1024.0 * 1024.0));
            return PI_OK;
        }
    }
    if (buf && n) snprintf(buf, n, "no gfx950 device among %d", count);
    return PI_E_HIP;
}

int pi_hip_create(pi_ctx **out, int device) {
    if (!out) return PI_E_INVALID;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return PI_E_HIP;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess) return PI_E_HIP;
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0) return PI_E_HIP;
    if (hipSetDevice(device) != hipSuccess) return PI_E_HIP;
    pi_ctx *c = new pi_ctx();
    c->device = device;
    if (hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return PI_E_HIP;
    }
    c->stream = c->own;
    c->scratch = scratch_init(device);
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeSharedMemPerBlockOptin, device) == hipSuccess && lds > 0)
        c->max_lds = lds;
    char buf[300];
    snprintf(buf, sizeof buf, "HIP %s (%s)", p.name, p.gcnArchName);
    c->name = buf;
    *out = c;
    return PI_OK;
}

void pi_hip_destroy(pi_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    engine_free(c->eng);
    pi_hip_clear_weight_cache(c);
    for (void *p : {(void *)c->io_x, (void *)c->io_y, (void *)c->io_q, (void *)c->io_d, (void *)c->io_s}) dfree(p);
    if (c->own) (void)hipStreamDestroy(c->own);
    delete c;
}

const char *pi_hip_name(const pi_ctx *c) { return c ? c->name.c_str() : ""; }
const char *pi_last_error(const pi_ctx *c) { return c ? c->err.c_str() : "no context"; }

int pi_hip_supports(const pi_ctx *c, uint32_t t) { return c && (pi_gemv_type(t) || pi_row_type(t)) ? 1 : 0; }

void pi_hip_clear_weight_cache(pi_ctx *c) {
    if (!c) return;
    for (auto &kv : c->wcache) free_tensor(kv.second);
    c->wcache.clear();
}

int pi_hip_set_stream(pi_ctx *c, void *s) {
    if (!c) return PI_E_INVALID;
    c->stream = s ? (hipStream_t)s : c->own;
    return PI_OK;
}

int pi_hip_synchronize(pi_ctx *c) {
    if (!c) return PI_E_INVALID;
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

int pi_hip_use_graphs(pi_ctx *c, int enable) {
    if (!c) return PI_E_INVALID;
    c->use_graphs = enable != 0;
    return PI_OK;
}

int pi_hip_use_persistent(pi_ctx *c, int enable) {
    if (!c) return PI_E_INVALID;
    c->use_persistent = enable != 0;
    return PI_OK;
}

int pi_hip_use_batch_prefill(pi_ctx *c, int enable) {
    if (!c) return PI_E_INVALID;
    c->use_batch_prefill = enable != 0;
    return PI_OK;
}

int pi_hip_persistent_active(const pi_ctx *c) { return c && c->eng && use_mega(c, *c->eng) ? 1 : 0; }

int pi_hip_prefill_pass_tokens(const pi_ctx *c) { return c && c->eng && c->eng->pf_ok ? (int)c->eng->pf_pass : 0; }

int pi_hip_stage_trace(pi_ctx *c, int enable) {
    if (!c) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e) return fail(c, PI_E_NOMODEL, "no model bound");
    if (!e->mega_ok) return fail(c, PI_E_UNSUPPORTED, "the bound model does not run on the persistent kernel");
    HIPC(c, hipStreamSynchronize(c->stream));
    if (enable && !e->mega_trace) {
        const size_t n = (size_t)e->mega_blocks * pi_mega_trace_slots(e->n_layer);
        int r = dalloc(c, &e->mega_trace, n);
        if (r) return r;
        HIPC(c, hipMemset(e->mega_trace, 0, n * 8));
    }
    e->mega.trace = enable ? e->mega_trace : nullptr;
    HIPC(c, hipMemcpy(e->mega_dev, &e->mega, sizeof e->mega, hipMemcpyHostToDevice));
    return PI_OK;
}

int pi_hip_stage_trace_read(pi_ctx *c, uint64_t *out, size_t n, uint32_t *blocks, uint32_t *slots) {
    if (!c || !blocks || !slots) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e || !e->mega_trace) return fail(c, PI_E_INVALID, "stage tracing is off");
    *blocks = e->mega_blocks;
    *slots = pi_mega_trace_slots(e->n_layer);
    const size_t need = (size_t)*blocks * *slots;
    if (!out) return PI_OK;
    if (n < need) return fail(c, PI_E_INVALID, "trace needs %zu entries", need);
    HIPC(c, hipStreamSynchronize(c->stream));
    HIPC(c, hipMemcpy(out, e->mega_trace, need * 8, hipMemcpyDeviceToHost));
    return PI_OK;
}

int pi_hip_fail_next(pi_ctx *c) {
    if (!c) return PI_E_INVALID;
    c->fail_next = true;
    return PI_OK;
}

int pi_hip_upload(pi_ctx *c, uint32_t type, const void *host, size_t rows, size_t k, pi_tensor **out) {
    if (!c || !out) return PI_E_INVALID;
    return upload_tensor(c, type, host, rows, k, out);
}

void pi_hip_tensor_free(pi_ctx *c, pi_tensor *t) {
    (void)c;
    free_tensor(t);
}

size_t pi_hip_tensor_bytes(const pi_tensor *t) { return t ? (size_t)t->L.bytes : 0; }

int pi_hip_gemv_q8_dev(pi_ctx *c, const pi_tensor *w, const int8_t *q, const float *d, const int32_t *s, float *y) {
    if (!c || !w || !q || !d || !s || !y) return PI_E_INVALID;
    if (!pi_gemv_type(w->L.type)) return fail(c, PI_E_UNSUPPORTED, "type %u has no int8 path", w->L.type);
    if (take_injected(c)) return PI_E_INJECTED;
    HIPC(c, launch_single_gemv(w, q, d, s, y, nullptr, PI_GEMV_OUT, c->stream));
    return PI_OK;
}

// y = W x for an f32 x in HBM (the whole job of pi_hip_gemv_dev): one
// launch whose workgroups each quantize x into LDS; for rows too long for
// that LDS, Q8 of x into the context's staging buffers, then the GEMV.
static int enqueue_gemv_x(pi_ctx *c, const pi_tensor *w, const float *x, float *y) {
    if (pi_row_type(w->L.type)) {
        HIPC(c, pi_launch_gemv_row(w->L.type, w->dev, pi_row_bytes(w->L.type, w->L.k), w->L.rows, w->L.k, x, y, c->stream));
        return PI_OK;
    }
    if (pi_gemv_x_lds_bytes(w->L.type, w->L.g, w->L.k) <= (size_t)c->max_lds) {
        const pi_matset M = make_set({{w, y}});
        HIPC(c, pi_launch_gemv_x(M, x, gemv_blocks(w->L.ntiles), c->stream));
        return PI_OK;
    }
    int r = grow_io(c, w->L.k, 1);
    if (r) return r;
    HIPC(c, pi_launch_q8(x, w->L.k, 1, c->io_q, c->io_d, c->io_s, c->stream));
    HIPC(c, launch_single_gemv(w, c->io_q, c->io_d, c->io_s, y, nullptr, PI_GEMV_OUT, c->stream));
    return PI_OK;
}

int pi_hip_gemv_dev(pi_ctx *c, const pi_tensor *w, const float *x, float *y) {
    if (!c || !w || !x || !y) return PI_E_INVALID;
    if (take_injected(c)) return PI_E_INJECTED;
    return enqueue_gemv_x(c, w, x, y);
}

int pi_hip_q8_quantize_dev(pi_ctx *c, const float *x, size_t k, int b, int8_t *q, float *d, int32_t *s) {
    if (!c || !x || !q || !d || !s || k == 0 || k % 32 || b < 1 || b > 64) return PI_E_INVALID;
    HIPC(c, pi_launch_q8(x, (uint32_t)k, (uint32_t)b, q, d, s, c->stream));
    return PI_OK;
}

int pi_hip_dev_alloc(pi_ctx *c, size_t bytes, void **out) {
    if (!c || !out) return PI_E_INVALID;
    *out = nullptr;
    HIPC(c, hipSetDevice(c->device));
    hipError_t e = hipMalloc(out, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(c, PI_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return PI_OK;
}

void pi_hip_dev_free(pi_ctx *c, void *p) {
    (void)c;
    dfree(p);
}

int pi_hip_copy_h2d(pi_ctx *c, void *dst, const void *src, size_t bytes) {
    if (!c || !dst || !src) return PI_E_INVALID;
    HIPC(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

int pi_hip_copy_d2d(pi_ctx *c, void *dst, const void *src, size_t bytes) {
    if (!c || !dst || !src) return PI_E_INVALID;
    size_t bulk = 0;
    if ((((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
        bulk = bytes & ~(size_t)15;
        HIPC(c, pi_launch_copy16(src, dst, bulk / 16, c->stream));
    }
    if (bytes > bulk)
        HIPC(c, hipMemcpyAsync((uint8_t *)dst + bulk, (const uint8_t *)src + bulk, bytes - bulk,
                               hipMemcpyDeviceToDevice, c->stream));
    return PI_OK;
}

int pi_hip_copy_d2h(pi_ctx *c, void *dst, const void *src, size_t bytes) {
    if (!c || !dst || !src) return PI_E_INVALID;
    HIPC(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

int pi_hip_time_gemv(pi_ctx *c, const pi_tensor *const *ws, int n_copies, const int8_t *q, const float *d,
                     const int32_t *s, float *y, int iters, double *avg_us) {
    if (!c || !ws || n_copies < 1 || iters < 1 || !avg_us) return PI_E_INVALID;
    for (int i = 0; i < n_copies; i++)
        if (!ws[i] || !pi_gemv_type(ws[i]->L.type)) return fail(c, PI_E_UNSUPPORTED, "time_gemv: int8-path types only");
    hipEvent_t a, b;
    HIPC(c, hipEventCreate(&a));
    HIPC(c, hipEventCreate(&b));
    HIPC(c, hipEventRecord(a, c->stream));
    for (int i = 0; i < iters; i++) {
        const pi_tensor *w = ws[i % n_copies];
        HIPC(c, launch_single_gemv(w, q, d, s, y, nullptr, PI_GEMV_OUT, c->stream));
    }
    HIPC(c, hipEventRecord(b, c->stream));
    HIPC(c, hipEventSynchronize(b));
    float ms = 0.f;
    HIPC(c, hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *avg_us = (double)ms * 1000.0 / iters;
    return PI_OK;
}

int pi_hip_time_gemv_x(pi_ctx *c, const pi_tensor *const *ws, int n_copies, const float *x, float *y, int iters,
                       double *avg_us) {
    if (!c || !ws || n_copies < 1 || iters < 1 || !x || !y || !avg_us) return PI_E_INVALID;
    for (int i = 0; i < n_copies; i++)
        if (!ws[i] || ws[i]->L.k != ws[0]->L.k) return fail(c, PI_E_INVALID, "weight copies differ in row length");
    int r = grow_io(c, ws[0]->L.k, 1);
    if (r) return r;
    hipEvent_t a, b;
    HIPC(c, hipEventCreate(&a));
    HIPC(c, hipEventCreate(&b));
    HIPC(c, hipEventRecord(a, c->stream));
    for (int i = 0; i < iters; i++)
        if ((r = enqueue_gemv_x(c, ws[i % n_copies], x, y))) return r;
    HIPC(c, hipEventRecord(b, c->stream));
    HIPC(c, hipEventSynchronize(b));
    float ms = 0.f;
    HIPC(c, hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *avg_us = (double)ms * 1000.0 / iters;
    return PI_OK;
}

int pi_hip_matvec(pi_ctx *c, uint32_t type, const uint8_t *w, size_t w_bytes, size_t k, const float *x, float *out,
                  size_t rows) {
    if (!c || !w || !x || !out || rows == 0 || k == 0) return c ? fail(c, PI_E_INVALID, "invalid matvec arguments") : PI_E_INVALID;
    if (take_injected(c)) return PI_E_INJECTED;
    if (!pi_gemv_type(type) && !pi_row_type(type)) return fail(c, PI_E_UNSUPPORTED, "type not supported");
    if (pi_row_bytes(type, k) * rows != w_bytes)
        return fail(c, PI_E_INVALID, "weight bytes %zu do not match %zu rows of k=%zu", w_bytes, rows, k);
    auto key = std::make_pair((uintptr_t)w, w_bytes);
    pi_tensor *t;
    auto it = c->wcache.find(key);
    if (it != c->wcache.end() && it->second->L.k == k && it->second->L.type == type) {
        t = it->second;
    } else {
        if (it != c->wcache.end()) { free_tensor(it->second); c->wcache.erase(it); }
        int r = upload_tensor(c, type, w, rows, k, &t);
        if (r) return r;
        c->wcache[key] = t;
    }
    int r = grow_io(c, k, rows);
    if (r) return r;
    HIPC(c, hipMemcpyAsync(c->io_x, x, k * 4, hipMemcpyHostToDevice, c->stream));
    if ((r = enqueue_gemv_x(c, t, c->io_x, c->io_y))) return r;
    HIPC(c, hipMemcpyAsync(out, c->io_y, rows * 4, hipMemcpyDeviceToHost, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

int pi_hip_matvec_noalloc(pi_ctx *c, const pi_tensor *w, const float *x, float *out) {
    if (!c || !w || !x || !out) return c ? fail(c, PI_E_INVALID, "invalid matvec_noalloc arguments") : PI_E_INVALID;
    if (take_injected(c)) return PI_E_INJECTED;
    const size_t k = w->L.k, rows = w->L.rows;
    if (k > PI_NOALLOC_MAX_K || rows > PI_NOALLOC_MAX_ROWS)
        return fail(c, PI_E_INVALID, "matvec_noalloc: %zu rows x %zu exceeds the static staging (%u rows, k %u)",
                    rows, k, (unsigned)PI_NOALLOC_MAX_ROWS, (unsigned)PI_NOALLOC_MAX_K);
    if (!c->scratch) {
        const hipError_t e = (c->device >= 0 && c->device < kMaxDevices) ? g_scratch_err[c->device] : hipErrorInvalidDevice;
        return fail(c, PI_E_HIP, "matvec_noalloc: no staging address for device %d: %s", c->device, hipGetErrorString(e));
    }
    const bool row = pi_row_type(w->L.type);
    if (!row && pi_gemv_x_lds_bytes(w->L.type, w->L.g, w->L.k) > (size_t)c->max_lds)
        return fail(c, PI_E_UNSUPPORTED, "matvec_noalloc: row length %zu does not fit the kernel's LDS", k);
    float *xs = reinterpret_cast<float *>(c->scratch);
    float *ys = xs + PI_NOALLOC_MAX_K;
    HIPC(c, hipMemcpyAsync(xs, x, k * 4, hipMemcpyHostToDevice, c->stream));
    if (row) {
        HIPC(c, pi_launch_gemv_row(w->L.type, w->dev, pi_row_bytes(w->L.type, k), (uint32_t)rows, (uint32_t)k, xs, ys,
                                   c->stream));
    } else {
        const pi_matset M = make_set({{w, ys}});
        HIPC(c, pi_launch_gemv_x(M, xs, gemv_blocks(w->L.ntiles), c->stream));
    }
    HIPC(c, hipMemcpyAsync(out, ys, rows * 4, hipMemcpyDeviceToHost, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

int pi_hip_selftest(pi_ctx *c) {
    if (!c) return PI_E_INVALID;
    const size_t k = 256;
    float x[256];
    for (size_t j = 0; j < k; j++) x[j] = (float)(j % 7) * 0.1f - 0.3f;
    uint8_t w4[144] = {0};
    w4[0] = 0x00; w4[1] = 0x3C;  // d = 1.0
    w4[4] = 1;
    for (int i = 0; i < 128; i++) w4[16 + i] = 0x21;
    float out4 = 0.f;
    int r = pi_hip_matvec(c, PI_TYPE_Q4_K, w4, sizeof w4, k, x, &out4, 1);
    if (r) { pi_hip_clear_weight_cache(c); return r; }
    float want4 = selftest_dot_q4k(w4, x);
    if (std::fabs(out4 - want4) > std::fabs(want4) * 0.02f + 0.01f) {
        pi_hip_clear_weight_cache(c);
        return fail(c, PI_E_SELFTEST, "q4_K self-test failed: gpu=%g cpu=%g", out4, want4);
    }
    uint8_t w6[210] = {0};
    for (int i = 0; i < 128; i++) w6[i] = 0x95;
    for (int i = 0; i < 64; i++) w6[128 + i] = 0x1B;
    for (int i = 0; i < 16; i++) w6[192 + i] = 2;
    w6[208] = 0x00; w6[209] = 0x3C;
    float out6 = 0.f;
    r = pi_hip_matvec(c, PI_TYPE_Q6_K, w6, sizeof w6, k, x, &out6, 1);
    if (r) { pi_hip_clear_weight_cache(c); return r; }
    float want6 = selftest_dot_q6k(w6, x);
    if (std::fabs(out6 - want6) > std::fabs(want6) * 0.02f + 0.01f) {
        pi_hip_clear_weight_cache(c);
        return fail(c, PI_E_SELFTEST, "q6_K self-test failed: gpu=%g cpu=%g", out6, want6);
    }
    pi_hip_clear_weight_cache(c);
    return PI_OK;
}

int pi_hip_q8_quantize(pi_ctx *c, const float *x, size_t k, int b, int8_t *q, float *d, int32_t *sum) {
    if (!c || !x || !q || !d || !sum || k == 0 || k % 32 || b < 1 || b > 64) return PI_E_INVALID;
    if (take_injected(c)) return PI_E_INJECTED;
    float *dx = nullptr;
    int8_t *dq = nullptr;
    float *dd = nullptr;
    int32_t *ds = nullptr;
    size_t n = k * (size_t)b, nb = k / 32 * (size_t)b;
    int r;
    if ((r = dalloc(c, &dx, n)) || (r = dalloc(c, &dq, n)) || (r = dalloc(c, &dd, nb)) || (r = dalloc(c, &ds, nb))) {
        dfree(dx); dfree(dq); dfree(dd); dfree(ds);
        return r;
    }
    hipError_t e = hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = pi_launch_q8(dx, (uint32_t)k, (uint32_t)b, dq, dd, ds, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(q, dq, n, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(d, dd, nb * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(sum, ds, nb * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    dfree(dx); dfree(dq); dfree(dd); dfree(ds);
    if (e != hipSuccess) return fail(c, PI_E_HIP, "q8_quantize: %s", hipGetErrorString(e));
    return PI_OK;
}

int pi_hip_block_sums(pi_ctx *c, const pi_tensor *w, const int8_t *q, const float *d, const int32_t *sum,
                      int32_t *sums) {
    if (!c || !w || !q || !d || !sum || !sums) return PI_E_INVALID;
    if (take_injected(c)) return PI_E_INJECTED;
    const size_t k = w->L.k, nb = k / 32;
    const size_t per_row = (w->L.type == PI_TYPE_Q6_K) ? k / 16 : k / 32;
    const size_t n = per_row * w->L.rows;
    int32_t *dsums = nullptr;
    int r = grow_io(c, k, 1);
    if (r) return r;
    if ((r = dalloc(c, &dsums, n))) return r;
    hipError_t e = hipMemcpyAsync(c->io_q, q, k, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(c->io_d, d, nb * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(c->io_s, sum, nb * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess)
        e = launch_single_gemv(w, c->io_q, c->io_d, c->io_s, nullptr, dsums, PI_GEMV_SUMS, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(sums, dsums, n * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    dfree(dsums);
    if (e != hipSuccess) return fail(c, PI_E_HIP, "block_sums: %s", hipGetErrorString(e));
    return PI_OK;
}

// ---------------------------------------------------------------------------
// Engine entry points
// ---------------------------------------------------------------------------
int pi_hip_model_bind(pi_ctx *c, const pi_model_desc *m, uint32_t n_ctx) {
    if (!c || !m || !m->layers || n_ctx == 0) return c ? fail(c, PI_E_INVALID, "invalid model descriptor") : PI_E_INVALID;
    engine_free(c->eng);
    c->eng = nullptr;
    // Config::from_gguf / Model::finish checks (model.rs:43-81, 571-601)
    if (m->n_layer == 0 || m->n_embd == 0 || m->n_ff == 0 || m->n_head == 0)
        return fail(c, PI_E_INVALID, "invalid model configuration: zero layer, hidden, FFN or head count");
    if (m->head_dim == 0 || m->n_head_kv == 0 || m->n_head % m->n_head_kv)
        return fail(c, PI_E_INVALID, "invalid GQA configuration");
    if (m->n_rot == 0 || m->n_rot > m->head_dim || m->n_rot % 2 || !std::isfinite(m->rope_theta) || m->rope_theta <= 0.f ||
        !std::isfinite(m->rms_eps) || m->rms_eps <= 0.f)
        return fail(c, PI_E_INVALID, "invalid RoPE / RMSNorm configuration");
    if (m->head_dim != 64) return fail(c, PI_E_UNSUPPORTED, "attention kernel supports head_dim 64 (got %u)", m->head_dim);
    if (m->n_embd % 32 || m->n_ff % 32) return fail(c, PI_E_UNSUPPORTED, "hidden and FFN sizes must be multiples of 32");
    const uint64_t ne = m->n_embd, vocab = m->token_embd.ne1;
    const uint64_t qdim = (uint64_t)m->n_head * m->head_dim, kdim = (uint64_t)m->n_head_kv * m->head_dim;
    if (qdim != ne) return fail(c, PI_E_UNSUPPORTED, "n_head*head_dim must equal n_embd");
    if (vocab == 0 || m->token_embd.ne0 != ne || (m->n_vocab && m->n_vocab != vocab))
        return fail(c, PI_E_INVALID, "embedding / metadata / tokenizer vocab dimensions disagree");
    if (!check_shape(m->output, ne, vocab) || !check_shape(m->output_norm, ne, 1))
        return fail(c, PI_E_INVALID, "output tensor shape mismatch");
    for (uint32_t l = 0; l < m->n_layer; l++) {
        const pi_layer_desc &L = m->layers[l];
        if (!check_shape(L.attn_norm, ne, 1) || !check_shape(L.ffn_norm, ne, 1) || !check_shape(L.attn_q, ne, qdim) ||
            !check_shape(L.attn_k, ne, kdim) || !check_shape(L.attn_v, ne, kdim) || !check_shape(L.attn_o, qdim, ne) ||
            !check_shape(L.ffn_gate, ne, m->n_ff) || !check_shape(L.ffn_up, ne, m->n_ff) ||
            !check_shape(L.ffn_down, m->n_ff, ne))
            return fail(c, PI_E_INVALID, "layer %u tensor shape mismatch", l);
    }
    // token_embd rows are dequantized on the device (embed_elem)
    if (m->token_embd.type != PI_TYPE_F32 && !pi_gemv_type(m->token_embd.type))
        return fail(c, PI_E_UNSUPPORTED, "token_embd type %u unsupported", m->token_embd.type);
    // kernel coverage: Q/K (and gate/up, and the head) are super-block types
    // with a fused norm prologue; V may differ from Q/K only between Q4_K and
    // Q6_K; O and down take any GEMV type.
    auto kq = [](uint32_t t) { return t == PI_TYPE_Q4_K || t == PI_TYPE_Q6_K; };
    if (!kq(m->output.type)) return fail(c, PI_E_UNSUPPORTED, "output type %u: the head GEMV needs Q4_K or Q6_K", m->output.type);
    for (uint32_t l = 0; l < m->n_layer; l++) {
        const pi_layer_desc &L = m->layers[l];
        if (!kq(L.attn_q.type) || L.attn_k.type != L.attn_q.type || !kq(L.attn_v.type))
            return fail(c, PI_E_UNSUPPORTED, "layer %u: attn_q/attn_k/attn_v types %u/%u/%u not supported", l,
                        L.attn_q.type, L.attn_k.type, L.attn_v.type);
        if (!kq(L.ffn_gate.type) || L.ffn_up.type != L.ffn_gate.type)
            return fail(c, PI_E_UNSUPPORTED, "layer %u: ffn_gate/ffn_up types %u/%u not supported", l, L.ffn_gate.type,
                        L.ffn_up.type);
        if (!pi_gemv_type(L.attn_o.type) || !pi_gemv_type(L.ffn_down.type))
            return fail(c, PI_E_UNSUPPORTED, "layer %u: attn_o/ffn_down types %u/%u not supported", l, L.attn_o.type,
                        L.ffn_down.type);
    }
    {
        int dev = 0, maxlds = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&maxlds, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess || maxlds <= 0)
            maxlds = 65536;
        if (pi_attn_lds_bytes(n_ctx) > (size_t)maxlds)
            return fail(c, PI_E_UNSUPPORTED, "n_ctx %u needs %zu bytes of LDS for attention (device has %d)", n_ctx,
                        pi_attn_lds_bytes(n_ctx), maxlds);
    }
    Engine *e = new Engine();
    e->n_layer = m->n_layer; e->n_embd = m->n_embd; e->n_ff = m->n_ff; e->n_head = m->n_head;
    e->n_kv = m->n_head_kv; e->dh = m->head_dim; e->n_rot = m->n_rot; e->n_vocab = (uint32_t)vocab;
    e->eps = m->rms_eps; e->theta = m->rope_theta; e->n_ctx = n_ctx;
    e->eos.assign(m->eos_ids, m->eos_ids + m->n_eos);
    e->layers.resize(m->n_layer);
    int r = PI_OK;
#define TRY(expr) do { if ((r = (expr)) != PI_OK) { engine_free(e); return r; } } while (0)
    for (uint32_t l = 0; l < m->n_layer; l++) {
        const pi_layer_desc &D = m->layers[l];
        Layer &L = e->layers[l];
        TRY(upload_mat(c, D.attn_q, &L.q));
        TRY(upload_mat(c, D.attn_k, &L.k));
        TRY(upload_mat(c, D.attn_v, &L.v));
        TRY(upload_mat(c, D.attn_o, &L.o));
        TRY(upload_mat(c, D.ffn_gate, &L.gate));
        TRY(upload_mat(c, D.ffn_up, &L.up));
        TRY(upload_mat(c, D.ffn_down, &L.down));
        TRY(upload_norm(c, D.attn_norm, e->n_embd, &L.attn_norm));
        TRY(upload_norm(c, D.ffn_norm, e->n_embd, &L.ffn_norm));
    }
    TRY(upload_mat(c, m->output, &e->head));
    TRY(upload_norm(c, m->output_norm, e->n_embd, &e->out_norm));
    e->embd_type = m->token_embd.type;
    e->embd_row_bytes = pi_row_bytes(e->embd_type, ne);
    if (e->embd_row_bytes == 0) { engine_free(e); return fail(c, PI_E_UNSUPPORTED, "token_embd row length"); }
    TRY(dalloc(c, &e->embd, e->embd_row_bytes * vocab));
    if (hipMemcpy(e->embd, m->token_embd.data, e->embd_row_bytes * vocab, hipMemcpyHostToDevice) != hipSuccess) {
        engine_free(e);
        return fail(c, PI_E_HIP, "token_embd upload failed");
    }
    // KV cache [layer][kv_head][n_ctx][head_dim] f32, zeroed (model.rs:362-373)
    const uint64_t nkv = (uint64_t)e->n_layer * e->n_kv * n_ctx * e->dh;
    TRY(dalloc(c, &e->kc, nkv));
    TRY(dalloc(c, &e->vc, nkv));
    if (hipMemset(e->kc, 0, nkv * 4) != hipSuccess || hipMemset(e->vc, 0, nkv * 4) != hipSuccess) {
        engine_free(e);
        return fail(c, PI_E_HIP, "KV clear failed");
    }
    // RoPE tables (model.rs:413-417, 445-460), host libm like the reference
    const uint32_t half = e->n_rot / 2;
    std::vector<float> inv(half), ct((size_t)n_ctx * half), stt((size_t)n_ctx * half);
    for (uint32_t i = 0; i < half; i++) inv[i] = 1.0f / pi_powf(e->theta, 2.0f * (float)i / (float)e->n_rot);
    for (uint32_t p = 0; p < n_ctx; p++)
        for (uint32_t i = 0; i < half; i++) {
            float a = (float)p * inv[i];
            ct[(size_t)p * half + i] = pi_cosf(a);
            stt[(size_t)p * half + i] = pi_sinf(a);
        }
    TRY(dalloc(c, &e->cos_tab, ct.size()));
    TRY(dalloc(c, &e->sin_tab, stt.size()));
    if (hipMemcpy(e->cos_tab, ct.data(), ct.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(e->sin_tab, stt.data(), stt.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        engine_free(e);
        return fail(c, PI_E_HIP, "RoPE table upload failed");
    }
    const uint32_t big = e->n_embd > e->n_ff ? e->n_embd : e->n_ff;
    TRY(dalloc(c, &e->x, ne)); TRY(dalloc(c, &e->q, qdim)); TRY(dalloc(c, &e->k, kdim)); TRY(dalloc(c, &e->v, kdim));
    TRY(dalloc(c, &e->h, e->n_ff));
    TRY(dalloc(c, &e->logits, vocab));
    TRY(dalloc(c, &e->amax_v, PI_HEAD_BLOCKS)); TRY(dalloc(c, &e->amax_i, PI_HEAD_BLOCKS));
    TRY(dalloc(c, &e->ids, (size_t)n_ctx + kDecodeChunk + 2)); TRY(dalloc(c, &e->prompt, (size_t)n_ctx + 1));
    TRY(dalloc(c, &e->q8q, big)); TRY(dalloc(c, &e->q8d, big / 32)); TRY(dalloc(c, &e->q8s, big / 32));
    TRY(dalloc(c, &e->st, 1));
    if (hipMemset(e->logits, 0, vocab * 4) != hipSuccess) { engine_free(e); return fail(c, PI_E_HIP, "memset"); }
    TRY(build_graphs(c, *e));
    TRY(build_mega(c, *e));
    TRY(build_prefill(c, *e));
#undef TRY
    c->eng = e;
    return PI_OK;
}

static int forward_impl(pi_ctx *c, const uint32_t *ids, const int32_t *pos, int b, int want_logits, bool cancellable) {
    Engine *e = c->eng;
    if (b < 1 || (uint32_t)b > kMaxBatch) return fail(c, PI_E_INVALID, "invalid batch %d", b);
    for (int i = 0; i < b; i++) {
        if (pos[i] < 0 || (uint32_t)pos[i] >= e->n_ctx) return fail(c, PI_E_CONTEXT_FULL, "context full");
        if (ids[i] >= e->n_vocab) return fail(c, PI_E_INVALID, "token %u out of vocab", ids[i]);
        if (i > 0 && pos[i] <= pos[i - 1]) return fail(c, PI_E_INVALID, "batch positions must increase");
    }
    bool consecutive = true;
    for (int i = 1; i < b; i++) consecutive &= pos[i] == pos[0] + i;
    if (b > 1 && consecutive && use_pf(c, *e)) {
        // a batch of more than one token: every token in the multi-token
        // orders, in passes of at most pf_pass tokens on the batched kernels
        if (want_logits) {
            int r = set_state(c, *e, pos[b - 1], ids[b - 1], 0, 0);
            if (r) return r;
        }
        uint32_t last_nt = 0;
        for (int off = 0; off < b; off += (int)e->pf_pass) {
            if (cancellable && c->stop.load()) return fail(c, PI_E_STOPPED, "generation stopped");
            const uint32_t nt = std::min<uint32_t>(e->pf_pass, (uint32_t)(b - off));
            HIPC(c, hipMemcpyAsync(e->pf_ids, ids + off, nt * 4, hipMemcpyHostToDevice, c->stream));
            HIPC(c, pf_chunk(c, *e, e->pf_ids, (uint32_t)pos[off], nt));
            last_nt = nt;
        }
        if (want_logits) {
            HIPC(c, hipMemcpyAsync(e->x, e->pfX + (uint64_t)(last_nt - 1) * e->n_embd, (size_t)e->n_embd * 4,
                                   hipMemcpyDeviceToDevice, c->stream));
            HIPC(c, enqueue_logits(*e, c->stream));
            HIPC(c, enqueue_step(*e, PI_STEP_ARGMAX, nullptr, c->stream));
        }
        HIPC(c, hipStreamSynchronize(c->stream));
        return PI_OK;
    }
    if (use_mega(c, *e)) {
        for (int i = 0; i < b; i++) {
            if (cancellable && c->stop.load()) return fail(c, PI_E_STOPPED, "generation stopped");
            HIPC(c, mega_token(c, *e, pos[i], ids[i], nullptr, nullptr, b == 1, want_logits && i == b - 1));
        }
        HIPC(c, hipStreamSynchronize(c->stream));
        return mega_check(c, *e);
    }
    for (int i = 0; i < b; i++) {
        if (cancellable && c->stop.load()) return fail(c, PI_E_STOPPED, "generation stopped");
        int r = set_state(c, *e, pos[i], ids[i], 0, 0);
        if (r) return r;
        HIPC(c, enqueue_step(*e, PI_STEP_EMBED, nullptr, c->stream));
        // a batch of more than one token evaluates in the scalar order (model.rs:812-822, 1028-1038)
        HIPC(c, run_step(c, *e, b > 1 ? STEP_LAYERS_SEQ : STEP_LAYERS_NEON));
    }
    if (want_logits) HIPC(c, run_step(c, *e, STEP_LOGITS));
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

int pi_hip_forward(pi_ctx *c, const uint32_t *ids, const int32_t *pos, int b, int want_logits) {
    if (!c) return PI_E_INVALID;
    if (!c->eng) return fail(c, PI_E_NOMODEL, "no model bound");
    if (!ids || !pos) return fail(c, PI_E_INVALID, "null ids/positions");
    if (take_injected(c)) return PI_E_INJECTED;
    // Engine::forward invalidates reuse (model.rs:825-831)
    c->eng->kv_tokens.clear();
    c->eng->cached_prefill_len = 0;
    return forward_impl(c, ids, pos, b, want_logits, false);
}

int pi_hip_logits(pi_ctx *c, float *out, size_t n) {
    if (!c || !out) return PI_E_INVALID;
    if (!c->eng) return fail(c, PI_E_NOMODEL, "no model bound");
    if (n > c->eng->n_vocab) return fail(c, PI_E_INVALID, "asked for %zu logits of %u", n, c->eng->n_vocab);
    HIPC(c, hipMemcpyAsync(out, c->eng->logits, n * 4, hipMemcpyDeviceToHost, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    return PI_OK;
}

int pi_hip_argmax(pi_ctx *c, uint32_t *id) {
    if (!c || !id) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e) return fail(c, PI_E_NOMODEL, "no model bound");
    // the persistent kernel leaves the greedy id of its last head in the state
    if (!use_mega(c, *e)) HIPC(c, enqueue_step(*e, PI_STEP_ARGMAX, nullptr, c->stream));
    pi_state h;
    HIPC(c, hipMemcpyAsync(&h, e->st, sizeof h, hipMemcpyDeviceToHost, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    *id = h.tok;
    return PI_OK;
}

void pi_hip_request_stop(pi_ctx *c) { if (c) c->stop.store(1); }
void pi_hip_clear_stop(pi_ctx *c) { if (c) c->stop.store(0); }

int pi_hip_last_decode_us(pi_ctx *c, double *us) {
    if (!c || !us || !c->eng) return PI_E_INVALID;
    *us = c->eng->last_decode_us;
    return PI_OK;
}

int pi_hip_time_kernels(pi_ctx *c, int enable) {
    if (!c) return PI_E_INVALID;
    c->time_kernels = enable != 0;
    return PI_OK;
}

int pi_hip_last_kernel_us(pi_ctx *c, double *us, uint32_t *n) {
    if (!c || !us || !n || !c->eng) return PI_E_INVALID;
    *us = c->eng->last_kernel_us;
    *n = c->eng->last_kernel_n;
    return PI_OK;
}

// Decode with temperature / top-p sampling (model.rs:1299-1337 with
// sampler.rs:21-92): after every forward the logits come back to the host,
// where the token is drawn from the seeded generator; the token then feeds
// the next forward.  The logits left on the device afterwards are the
// weights the last draw used, as sample() leaves them in the reference's
// scratch.logits.
static int sample_decode(pi_ctx *c, Engine &e, size_t n, const pi_genopts *o, pi_genstats *st, uint32_t *gen_ids,
                         bool mega) {
    int r;
    auto g0 = std::chrono::steady_clock::now();
    pi_rng rng = pi_rng_make(o->seed);
    std::vector<float> lg(e.n_vocab);
    std::vector<uint32_t> idx;
    hipEvent_t ka = nullptr, kb = nullptr;
    if (c->time_kernels) {
        HIPC(c, hipEventCreate(&ka));
        HIPC(c, hipEventCreate(&kb));
    }
    double kern_ms = 0.0;
    size_t fwd = 0;
    const size_t max_gen = o->max_tokens;
    for (size_t i = 0; i < max_gen; i++) {
        if (c->stop.load()) { snprintf(st->stop, sizeof st->stop, "user_stop"); break; }
        HIPC(c, hipMemcpyAsync(lg.data(), e.logits, (size_t)e.n_vocab * 4, hipMemcpyDeviceToHost, c->stream));
        HIPC(c, hipStreamSynchronize(c->stream));
        const uint32_t tok = pi_sample_logits(lg.data(), lg.size(), o->temp, o->top_p, rng, idx);
        bool eog = false;
        for (uint32_t x : e.eos) eog |= (x == tok);
        if (eog) { snprintf(st->stop, sizeof st->stop, "eog"); break; }
        gen_ids[st->gen_tokens++] = tok;
        if (i + 1 == max_gen) break;
        const size_t pos = n + i;
        if (pos >= e.n_ctx) { snprintf(st->stop, sizeof st->stop, "context_full"); break; }
        if (ka) HIPC(c, hipEventRecord(ka, c->stream));
        if (mega) {
            HIPC(c, mega_token(c, e, (int32_t)pos, tok, nullptr, nullptr, true, true));
        } else {
            if ((r = set_state(c, e, (int32_t)pos, tok, 0, 0))) return r;
            HIPC(c, enqueue_step(e, PI_STEP_EMBED, nullptr, c->stream));
            HIPC(c, run_step(c, e, STEP_DECODE));
        }
        if (kb) HIPC(c, hipEventRecord(kb, c->stream));
        HIPC(c, hipStreamSynchronize(c->stream));
        if ((r = mega_check(c, e))) { e.kv_tokens.clear(); e.cached_prefill_len = 0; return r; }
        if (ka) {
            float ms = 0.f;
            HIPC(c, hipEventElapsedTime(&ms, ka, kb));
            kern_ms += ms;
        }
        e.kv_tokens.push_back(tok);
        fwd++;
    }
    // the weights of the last draw stay in the logits, as in the reference
    if (st->gen_tokens || strcmp(st->stop, "eog") == 0)
        HIPC(c, hipMemcpy(e.logits, lg.data(), (size_t)e.n_vocab * 4, hipMemcpyHostToDevice));
    if (ka) (void)hipEventDestroy(ka);
    if (kb) (void)hipEventDestroy(kb);
    e.last_kernel_us = (c->time_kernels && fwd) ? kern_ms * 1000.0 / (double)fwd : 0.0;
    e.last_kernel_n = c->time_kernels ? (uint32_t)fwd : 0u;
    if (strcmp(st->stop, "user_stop") == 0) { e.kv_tokens.clear(); e.cached_prefill_len = 0; }
    st->gen_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - g0).count();
    e.last_decode_us = fwd ? st->gen_ms * 1000.0 / (double)fwd : 0.0;
    return PI_OK;
}

int pi_hip_generate(pi_ctx *c, const uint32_t *prompt, size_t n, const pi_genopts *o, pi_genstats *st,
                    uint32_t *gen_ids) {
    if (!c || !o || !st) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e) return fail(c, PI_E_NOMODEL, "no model bound");
    memset(st, 0, sizeof *st);
    snprintf(st->stop, sizeof st->stop, "max_tokens");
    if (n == 0 || !prompt) return fail(c, PI_E_INVALID, "empty prompt");
    if (!(o->temp == o->temp) || !(o->top_p == o->top_p)) return fail(c, PI_E_INVALID, "temp / top_p is NaN");
    if (o->max_tokens > 0 && !gen_ids) return fail(c, PI_E_INVALID, "gen_ids is null");
    if (take_injected(c)) return PI_E_INJECTED;
    for (size_t i = 0; i < n; i++)
        if (prompt[i] >= e->n_vocab) return fail(c, PI_E_INVALID, "token %u out of vocab", prompt[i]);
    if (n > e->n_ctx) return fail(c, PI_E_CONTEXT_FULL, "context full");
    auto t0 = std::chrono::steady_clock::now();
    const size_t chunk = 32;
    // Reuse rule of model.rs:1258-1268.  The device prefill evaluates every
    // token with the same kernels whatever the chunking, so full-chunk reuse
    // is exact here and stays enabled while this backend is active.
    size_t common = 0;
    while (common < e->kv_tokens.size() && common < n && e->kv_tokens[common] == prompt[common]) common++;
    size_t reused = std::min(std::min(common, e->cached_prefill_len), n - 1) / chunk * chunk;
    e->kv_tokens.resize(reused);
    e->cached_prefill_len = 0;
    st->prefill_cached_tokens = (uint32_t)reused;
    const bool mega = use_mega(c, *e);
    HIPC(c, hipMemcpyAsync(e->prompt, prompt, n * 4, hipMemcpyHostToDevice, c->stream));
    int r = set_state(c, *e, (int32_t)reused, prompt[reused], 0, (uint32_t)reused);
    if (r) return r;
    if (!mega) HIPC(c, enqueue_step(*e, PI_STEP_EMBED, nullptr, c->stream));
    size_t off = reused;
    bool stopped = false;
    // Prefill in 32-token chunks from `reused` (model.rs:1269-1288).  Tokens of
    // a chunk of more than one token take the scalar-order graph; the last
    // prompt token also computes logits and the first greedy id.
    const size_t last_chunk = (n - reused) % chunk == 0 ? chunk : (n - reused) % chunk;
    if (use_pf(c, *e)) {
        // Reference chunks of 32 from `reused`: every token of a chunk of more
        // than one token runs on the batched prefill kernels, in passes of up
        // to pf_pass tokens that may span several chunks; a chunk of one
        // (only the last can be) runs in the batch-1 order.  The last pass
        // also computes the logits and the first greedy id of its last token.
        const size_t batched_end = last_chunk == 1 ? n - 1 : n;
        while (off < n) {
            if (c->stop.load()) { stopped = true; break; }
            const size_t end = off < batched_end ? std::min<size_t>(batched_end, off + e->pf_pass) : n;
            const bool last = end == n;
            if (off >= batched_end) {
                if (mega) {
                    HIPC(c, mega_token(c, *e, (int32_t)off, prompt[off], nullptr, e->ids, true, true));
                } else {
                    if ((r = set_state(c, *e, (int32_t)off, prompt[off], 0, (uint32_t)off))) return r;
                    HIPC(c, enqueue_step(*e, PI_STEP_EMBED, nullptr, c->stream));
                    HIPC(c, run_step(c, *e, STEP_DECODE));
                }
            } else {
                if (last && (r = set_state(c, *e, (int32_t)(n - 1), prompt[n - 1], 0, (uint32_t)(n - 1)))) return r;
                HIPC(c, pf_chunk(c, *e, e->prompt + off, (uint32_t)off, (uint32_t)(end - off)));
                if (last) {
                    HIPC(c, hipMemcpyAsync(e->x, e->pfX + (uint64_t)(end - off - 1) * e->n_embd,
                                           (size_t)e->n_embd * 4, hipMemcpyDeviceToDevice, c->stream));
                    HIPC(c, enqueue_logits(*e, c->stream));
                    HIPC(c, enqueue_step(*e, PI_STEP_ARGMAX, e->ids, c->stream));
                }
            }
            HIPC(c, hipStreamSynchronize(c->stream));
            if ((r = mega_check(c, *e))) { e->kv_tokens.clear(); return r; }
            e->kv_tokens.insert(e->kv_tokens.end(), prompt + off, prompt + end);
            off = end;
        }
        if (stopped) {
            snprintf(st->stop, sizeof st->stop, "user_stop");
            st->prefill_tokens = (uint32_t)(off - reused);
            e->kv_tokens.clear();
            st->prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            return PI_OK;
        }
        goto prefill_done;
    }
    while (off + 1 < n) {
        if (c->stop.load()) { stopped = true; break; }
        size_t end = std::min(n - 1, off + chunk);
        for (size_t t = off; t < end; t++) {
            if (mega) HIPC(c, mega_token(c, *e, (int32_t)t, prompt[t], nullptr, nullptr, false, false));
            else HIPC(c, run_step(c, *e, STEP_PREFILL));
        }
        HIPC(c, hipStreamSynchronize(c->stream));
        if ((r = mega_check(c, *e))) { e->kv_tokens.clear(); return r; }
        e->kv_tokens.insert(e->kv_tokens.end(), prompt + off, prompt + end);
        off = end;
    }
    if (!stopped && c->stop.load()) stopped = true;
    if (stopped) {
        snprintf(st->stop, sizeof st->stop, "user_stop");
        st->prefill_tokens = (uint32_t)(off - reused);
        e->kv_tokens.clear();
        st->prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        return PI_OK;
    }
    if (mega) HIPC(c, mega_token(c, *e, (int32_t)(n - 1), prompt[n - 1], nullptr, e->ids, last_chunk == 1, true));
    else HIPC(c, run_step(c, *e, last_chunk > 1 ? STEP_LAST_SEQ : STEP_DECODE));
    HIPC(c, hipStreamSynchronize(c->stream));
    if ((r = mega_check(c, *e))) { e->kv_tokens.clear(); return r; }
    e->kv_tokens.push_back(prompt[n - 1]);
prefill_done:
    off = n;
    st->prefill_tokens = (uint32_t)(off - reused);
    st->prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    e->cached_prefill_len = n;
    if (o->temp > 0.0f) return sample_decode(c, *e, n, o, st, gen_ids, mega);
    // Decode: n tokens take n-1 forwards (model.rs:1299-1337).
    auto g0 = std::chrono::steady_clock::now();
    hipEvent_t ea, eb;
    HIPC(c, hipEventCreate(&ea));
    HIPC(c, hipEventCreate(&eb));
    HIPC(c, hipEventRecord(ea, c->stream));
    // ids[i] is the token sampled after i forwards; forward i+1 evaluates it.
    size_t launched = 0;
    std::vector<uint32_t> host_ids;
    const size_t max_gen = o->max_tokens;
    const size_t fwd_cap = max_gen > 0 ? max_gen - 1 : 0;     // `i + 1 == max_gen` breaks first
    const size_t ctx_cap = e->n_ctx > n ? e->n_ctx - n : 0;  // `pos >= n_ctx` stops
    const size_t want_fwd = std::min(fwd_cap, ctx_cap);
    size_t i = 0;
    bool done = (max_gen == 0);
    // Kernel timing: an event pair around every decode forward; the mean of
    // their elapsed times is the device time of one forward's kernels.
    std::vector<hipEvent_t> kev;
    if (c->time_kernels) {
        kev.resize(2 * kDecodeChunk, nullptr);
        for (hipEvent_t &x : kev) HIPC(c, hipEventCreate(&x));
    }
    double kern_ms = 0.0;
    auto free_kev = [&] {
        for (hipEvent_t x : kev)
            if (x) (void)hipEventDestroy(x);
        kev.clear();
    };
    // The first id comes from the prompt's last forward: it is checked before
    // any decode forward is launched, so an immediate EOG leaves that
    // forward's logits in place (as Engine::generate does, model.rs:1305-1306).
    if (!done) {
        uint32_t first = 0;
        HIPC(c, hipMemcpyAsync(&first, e->ids, 4, hipMemcpyDeviceToHost, c->stream));
        HIPC(c, hipStreamSynchronize(c->stream));
        for (uint32_t x : e->eos) done |= (x == first);
        if (done) snprintf(st->stop, sizeof st->stop, "eog");
    }
    while (!done) {
        // launch up to kDecodeChunk forwards ahead, then read the ids back
        size_t target = std::min(want_fwd, launched + kDecodeChunk);
        const size_t base = launched;
        while (launched < target) {
            if (!kev.empty()) HIPC(c, hipEventRecord(kev[2 * (launched - base)], c->stream));
            if (mega)
                HIPC(c, mega_token(c, *e, (int32_t)(n + launched), 0, &e->st->tok, e->ids + launched + 1, true, true));
            else HIPC(c, run_step(c, *e, STEP_DECODE));
            if (!kev.empty()) HIPC(c, hipEventRecord(kev[2 * (launched - base) + 1], c->stream));
            launched++;
        }
        host_ids.resize(launched + 1);
        HIPC(c, hipMemcpyAsync(host_ids.data(), e->ids, (launched + 1) * 4, hipMemcpyDeviceToHost, c->stream));
        HIPC(c, hipStreamSynchronize(c->stream));
        if ((r = mega_check(c, *e))) { free_kev(); e->kv_tokens.clear(); e->cached_prefill_len = 0; return r; }
        for (size_t j = 0; j < launched - base && !kev.empty(); j++) {
            float ms = 0.f;
            HIPC(c, hipEventElapsedTime(&ms, kev[2 * j], kev[2 * j + 1]));
            kern_ms += ms;
        }
        while (!done && i <= launched) {
            if (c->stop.load()) { snprintf(st->stop, sizeof st->stop, "user_stop"); done = true; break; }
            const uint32_t tok = host_ids[i];
            bool eog = false;
            for (uint32_t x : e->eos) eog |= (x == tok);
            if (eog) { snprintf(st->stop, sizeof st->stop, "eog"); done = true; break; }
            gen_ids[st->gen_tokens++] = tok;
            if (i + 1 == max_gen) { done = true; break; }
            if (n + i >= e->n_ctx) { snprintf(st->stop, sizeof st->stop, "context_full"); done = true; break; }
            e->kv_tokens.push_back(tok);  // forward i+1 (launched now or in the next round)
            i++;
        }
    }
    HIPC(c, hipEventRecord(eb, c->stream));
    HIPC(c, hipEventSynchronize(eb));
    float ms = 0.f;
    HIPC(c, hipEventElapsedTime(&ms, ea, eb));
    (void)hipEventDestroy(ea);
    (void)hipEventDestroy(eb);
    free_kev();
    e->last_decode_us = launched ? (double)ms * 1000.0 / (double)launched : 0.0;
    e->last_kernel_us = (c->time_kernels && launched) ? kern_ms * 1000.0 / (double)launched : 0.0;
    e->last_kernel_n = c->time_kernels ? (uint32_t)launched : 0u;
    // An EOG sampled after i >= 1 forwards may have been read after later
    // forwards were already launched.  Forward i (token i-1 at position
    // n+i-1) is evaluated again: it writes the same KV row bit for bit and
    // leaves the logits and greedy id that produced the EOG, which is what
    // Engine::generate leaves behind (model.rs:1299-1337).
    if (strcmp(st->stop, "eog") == 0 && i >= 1 && launched > i) {
        const int32_t p = (int32_t)(n + i - 1);
        const uint32_t tk = host_ids[i - 1];
        if (mega) {
            HIPC(c, mega_token(c, *e, p, tk, nullptr, nullptr, true, true));
        } else {
            if ((r = set_state(c, *e, p, tk, 0, 0))) return r;
            HIPC(c, enqueue_step(*e, PI_STEP_EMBED, nullptr, c->stream));
            HIPC(c, run_step(c, *e, STEP_DECODE));
        }
        HIPC(c, hipStreamSynchronize(c->stream));
        if ((r = mega_check(c, *e))) { e->kv_tokens.clear(); e->cached_prefill_len = 0; return r; }
    }
    // Forwards launched past an EOS or stop only wrote KV rows beyond the
    // recorded tokens; they are never read before being overwritten.
    e->kv_tokens.resize(std::min(e->kv_tokens.size(), n + (size_t)st->gen_tokens));
    if (strcmp(st->stop, "user_stop") == 0) { e->kv_tokens.clear(); e->cached_prefill_len = 0; }
    st->gen_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - g0).count();
    return PI_OK;
}

uint64_t pi_rng_new(uint64_t seed) { return pi_rng_make(seed).s; }

uint64_t pi_rng_next_u64(uint64_t *state) {
    if (!state) return 0;
    pi_rng r{*state};
    const uint64_t v = pi_rng_u64(r);
    *state = r.s;
    return v;
}

uint32_t pi_sample(float *logits, size_t n, float temp, float top_p, uint64_t *rng_state) {
    if (!logits || !rng_state) return 0;
    pi_rng r{*rng_state};
    std::vector<uint32_t> idx;
    const uint32_t tok = pi_sample_logits(logits, n, temp, top_p, r, idx);
    *rng_state = r.s;
    return tok;
}

int pi_hip_kv_write(pi_ctx *c, uint32_t layer, uint32_t h, uint32_t pos0, uint32_t n, const float *k, const float *v) {
    if (!c || !k || !v) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e) return fail(c, PI_E_NOMODEL, "no model bound");
    if (layer >= e->n_layer || h >= e->n_kv || (uint64_t)pos0 + n > e->n_ctx) return fail(c, PI_E_INVALID, "KV range");
    uint64_t off = (((uint64_t)layer * e->n_kv + h) * e->n_ctx + pos0) * e->dh;
    HIPC(c, hipMemcpy(e->kc + off, k, (size_t)n * e->dh * 4, hipMemcpyHostToDevice));
    HIPC(c, hipMemcpy(e->vc + off, v, (size_t)n * e->dh * 4, hipMemcpyHostToDevice));
    e->kv_tokens.clear();
    e->cached_prefill_len = 0;
    return PI_OK;
}

int pi_hip_kv_read(pi_ctx *c, uint32_t layer, uint32_t h, uint32_t pos0, uint32_t n, float *k, float *v) {
    if (!c || !k || !v) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e) return fail(c, PI_E_NOMODEL, "no model bound");
    if (layer >= e->n_layer || h >= e->n_kv || (uint64_t)pos0 + n > e->n_ctx) return fail(c, PI_E_INVALID, "KV range");
    uint64_t off = (((uint64_t)layer * e->n_kv + h) * e->n_ctx + pos0) * e->dh;
    HIPC(c, hipStreamSynchronize(c->stream));
    HIPC(c, hipMemcpy(k, e->kc + off, (size_t)n * e->dh * 4, hipMemcpyDeviceToHost));
    HIPC(c, hipMemcpy(v, e->vc + off, (size_t)n * e->dh * 4, hipMemcpyDeviceToHost));
    return PI_OK;
}

int pi_hip_kv_fill_normal(pi_ctx *c, uint32_t n, uint64_t seed) {
    if (!c) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e) return fail(c, PI_E_NOMODEL, "no model bound");
    if (n > e->n_ctx) return fail(c, PI_E_INVALID, "KV range");
    HIPC(c, pi_launch_kv_fill(e->kc, e->vc, e->n_layer * e->n_kv, e->n_ctx, e->dh, n, seed, c->stream));
    HIPC(c, hipStreamSynchronize(c->stream));
    e->kv_tokens.clear();
    e->cached_prefill_len = 0;
    return PI_OK;
}

int pi_hip_kv_set_tokens(pi_ctx *c, const uint32_t *ids, uint32_t n) {
    if (!c || (!ids && n)) return PI_E_INVALID;
    Engine *e = c->eng;
    if (!e) return fail(c, PI_E_NOMODEL, "no model bound");
    if (n > e->n_ctx) return fail(c, PI_E_INVALID, "KV range");
    e->kv_tokens.assign(ids, ids + n);
    e->cached_prefill_len = n;
    return PI_OK;
}

}  // extern "C"
