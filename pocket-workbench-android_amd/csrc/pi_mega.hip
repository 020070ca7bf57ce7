// Persistent decode kernel for gfx950: one cooperative launch = one token
// through every layer (model.rs:857-1170), one workgroup of 4 wavefronts per
// CU, all workgroups resident.
//
// Stages of a layer and who runs them:
//   S1  every workgroup: x -> RMSNorm + Q8 into LDS; Q/K/V tiles    -> q, k, v
//   S2  two workgroups per head (one per half of the dimensions; more
//       score segments at long contexts): RoPE, KV write, attention,
//       Q8                                                          -> att
//   S3  every workgroup: att -> LDS; attn_output tiles, x + proj    -> xb
//   S4  every workgroup: xb -> RMSNorm + Q8; gate/up tile pairs,
//       SwiGLU                                                       -> h
//   S5  every workgroup: h -> Q8; ffn_down tiles, xb + proj          -> xo
// then, with the head: xo -> output norm + Q8; head tiles -> logits and a
// per-workgroup (max, first index) pair; workgroup 0 reduces the pairs to the
// greedy id (sampler.rs:26-36).
//
// Hand-off: every output element is one 64-bit word (value bits | epoch
// << 32) stored with a device-scope atomic store; a consumer re-reads a word
// until it carries the launch's epoch.  Each layer has its own words, so a
// word is written once per launch and no stage can overwrite data another
// workgroup still reads.  Dependencies only point to earlier stages and every
// workgroup runs the stages in order, so with all workgroups resident
// (cooperative launch) every wait ends; each wait is also bounded and raises
// the abort flag when exceeded, after which every workgroup leaves.
//
// Each stage requests its first weight tile before it waits for its input,
// so the HBM latency of the weights overlaps the hand-off.  The GEMV core,
// Q8 rule and float orders are those of pi_gemv.h / pi_decode.hip, so the
// results are bit-identical to the CPU path.
#define PI_CHAIN_B 4   // per-row chains read 4 float4 ahead (the kernel is at its register limit)
#include <hip/hip_runtime.h>

#include <type_traits>

#include "pi_mega.h"

using namespace pig;

namespace {

constexpr uint32_t MT = 256;           // threads per workgroup
constexpr uint32_t MW = MT / 64;       // wavefronts per workgroup
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kChunk = 64;        // attention positions per product chunk
constexpr uint32_t kChunkPad = 68;     // floats per dimension row of a chunk (16-byte aligned)
constexpr uint32_t kRedFloats = 512;   // small LDS scratch
constexpr uint32_t kStripFloats = MW * 64 * 16;

// Row stride of the transposed x (floats).  The rows are followed by at least
// 48 more floats of the LDS plan (row padding, then the Q8 activation), which
// the norm's sum-of-squares chain reads ahead and ignores.
__host__ __device__ constexpr uint32_t xt_stride(uint32_t ne) { return ne / 8 + 4; }
__host__ __device__ constexpr uint32_t align16(uint32_t b) { return (b + 15u) & ~15u; }
__host__ __device__ constexpr uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// ---------------------------------------------------------------------------
// flag-tagged words
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t ll_get(const uint64_t *p) {
    return __hip_atomic_load(gst(const_cast<uint64_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_put(uint64_t *p, uint32_t bits, uint32_t epoch) {
    __hip_atomic_store(gst(p), ((uint64_t)epoch << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool aborted(const int32_t *f) {
    return __hip_atomic_load(gst(const_cast<int32_t *>(f)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void raise_abort(int32_t *f) {
    __hip_atomic_store(gst(f), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Re-reads p until it carries `epoch` (w: the last value read).  False when
// the spin bound is exceeded or another workgroup raised the abort flag.
__device__ __forceinline__ bool ll_wait(const uint64_t *p, uint32_t epoch, uint64_t &w, const int32_t *abort_flag) {
    uint32_t it = 0;
    while ((uint32_t)(w >> 32) != epoch) {
        ++it;
        if ((it & 63u) == 0 && (it > kSpinLimit || aborted(abort_flag))) return false;
        __builtin_amdgcn_s_sleep(1);
        w = ll_get(p);
    }
    return true;
}

// Every thread of the workgroup polls words tid, tid + MT, ... (U of them at
// a time).  Each round re-reads every word still missing, so words that
// arrive one after another cost one round trip together, not one each.
// dst(i, bits) stores word i.
template <int U, typename Dst>
__device__ __forceinline__ bool wg_poll(const uint64_t *src, uint32_t n, uint32_t epoch, const int32_t *abort_flag,
                                        Dst dst) {
    static_assert(U <= 32, "pending mask is 32 bits");
    for (uint32_t i0 = threadIdx.x; i0 < n; i0 += MT * U) {
        uint64_t w[U];
        uint32_t pending = 0;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t i = i0 + u * MT;
            if (i < n) {
                w[u] = ll_get(src + i);
                pending |= 1u << u;
            }
        }
        for (uint32_t it = 0;; ++it) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (((pending >> u) & 1u) && (uint32_t)(w[u] >> 32) == epoch) {
                    dst(i0 + u * MT, (uint32_t)w[u]);
                    pending &= ~(1u << u);
                }
            }
            if (!pending) break;
            if ((it & 63u) == 63u && (it > kSpinLimit || aborted(abort_flag))) return false;
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int u = 0; u < U; u++)
                if ((pending >> u) & 1u) w[u] = ll_get(src + i0 + u * MT);
        }
    }
    return true;
}

// Per-launch scalars handed to every stage.
struct Run {
    int32_t pos;
    uint32_t epoch;
    bool neon;    // batch-1 float orders (else the multi-token chunk orders)
    bool detail;  // record the in-stage trace points (middle layer)
};

// Scalar fields of the launch arguments, read once with scalar loads.
struct Cfg {
    const pi_mega_args *args;
    const pi_mega_layer *layers;
    uint32_t n_layer, ne, n_ff, n_head, n_kv, half, n_ctx, etype, t_head;
    float eps, scale;
    const float *cos_tab, *sin_tab, *out_norm;
    const uint8_t *embd;
    uint64_t erow_bytes;
    float *logits;
    uint64_t *part, *trace, *amax, *aexp;
    uint32_t *tok_state;
    int32_t *abort_flag;
};

__device__ __forceinline__ Cfg load_cfg(const pi_mega_args *ap) {
    Cfg c;
    c.args = ap;
    c.layers = cload(&ap->layers);
    c.n_layer = cload(&ap->n_layer); c.ne = cload(&ap->ne); c.n_ff = cload(&ap->n_ff);
    c.n_head = cload(&ap->n_head); c.n_kv = cload(&ap->n_kv); c.half = cload(&ap->half);
    c.n_ctx = cload(&ap->n_ctx); c.etype = cload(&ap->etype); c.t_head = cload(&ap->t_head);
    c.eps = cload(&ap->eps); c.scale = cload(&ap->scale);
    c.cos_tab = cload(&ap->cos_tab); c.sin_tab = cload(&ap->sin_tab); c.out_norm = cload(&ap->out_norm);
    c.embd = cload(&ap->embd); c.erow_bytes = cload(&ap->erow_bytes);
    c.logits = cload(&ap->logits); c.part = cload(&ap->part); c.trace = cload(&ap->trace);
    c.tok_state = cload(&ap->tok_state); c.abort_flag = cload(&ap->abort_flag);
    c.amax = cload(&ap->amax); c.aexp = cload(&ap->aexp);
    return c;
}

// Workgroup barrier that orders LDS only.  Every cross-wavefront exchange in
// this kernel goes through LDS (global hand-offs carry their own epoch), so
// the barriers never need to wait for in-flight global loads or stores, such
// as a weight tile requested before a stage's input has arrived.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Workgroup OR of a predicate: wavefront ballots through 4 LDS words.
__device__ __forceinline__ bool wg_any(bool pred, int32_t *vote) {
    const bool any = __ballot(pred) != 0;
    lds_barrier();  // earlier readers of the words are done
    if ((threadIdx.x & 63u) == 0) vote[threadIdx.x >> 6] = any ? 1 : 0;
    lds_barrier();
    return (vote[0] | vote[1] | vote[2] | vote[3]) != 0;
}

// s_waitcnt vmcnt(0): every global load of this wavefront has landed.  Used
// where that is already true (after a completed poll) so the compiler stops
// guarding each following LDS access with a wait for in-flight loads.
__device__ __forceinline__ void vm_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ float comp4(const float4 &v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }

// ---------------------------------------------------------------------------
// LDS of a workgroup
// ---------------------------------------------------------------------------
struct QAct {        // Q8 activation of k elements (quant_int.rs:3-14)
    uint32_t *qw;    // k/4 words of quants, 16-byte chunks in act_chunk order
    float *d;        // k/32 block scales
    int32_t *s;      // k/32 block sums
};

struct Lds {
    float *xt;       // residual x, transposed: x[8j + c] at xt[c * XT + j]
    uint32_t XT;
    QAct act;        // Q8 activation of the stage input
    float *hb;       // h staging, embedding row bytes, attention products
    float *strip;    // this wavefront's term strip (64 * 16 floats)
    float *red;      // scratch
    float *sc;       // attention scores (n_ctx)
    int32_t *vote;   // wg_any words
};

struct LdsPlan {
    uint32_t xt, act, hb, strips, red, sc, total;
};

__host__ __device__ inline LdsPlan lds_plan(uint32_t ne, uint32_t n_ff, uint32_t n_ctx) {
    LdsPlan p{};
    const uint32_t kmax = umax(ne, n_ff);
    p.xt = 0;
    p.act = p.xt + align16(8u * xt_stride(ne) * 4u);
    p.hb = p.act + align16(kmax + kmax / 32u * 8u);
    p.strips = p.hb + align16(umax(umax(n_ff, ne) * 4u, 2u * kChunk * kChunkPad * 4u));
    p.red = p.strips + kStripFloats * 4u;
    p.sc = p.red + kRedFloats * 4u;
    // whole chunks of e_p, then the chain reader's read-ahead
    p.total = p.sc + align16((n_ctx + kChunk - 1u) / kChunk * kChunk * 4u) + 256u;
    return p;
}

__device__ __forceinline__ Lds carve(unsigned char *smem, uint32_t ne, uint32_t n_ff, uint32_t n_ctx) {
    const LdsPlan p = lds_plan(ne, n_ff, n_ctx);
    Lds L;
    L.xt = reinterpret_cast<float *>(smem + p.xt);
    L.XT = xt_stride(ne);
    L.act.qw = reinterpret_cast<uint32_t *>(smem + p.act);
    L.hb = reinterpret_cast<float *>(smem + p.hb);
    L.strip = reinterpret_cast<float *>(smem + p.strips) + (threadIdx.x >> 6) * 64 * 16;
    L.red = reinterpret_cast<float *>(smem + p.red);
    L.vote = reinterpret_cast<int32_t *>(L.red + kRedFloats - 8);
    L.sc = reinterpret_cast<float *>(smem + p.sc);
    return L;
}
__device__ __forceinline__ void set_act_k(Lds &L, uint32_t k) {
    L.act.d = reinterpret_cast<float *>(reinterpret_cast<unsigned char *>(L.act.qw) + k);
    L.act.s = reinterpret_cast<int32_t *>(reinterpret_cast<unsigned char *>(L.act.qw) + k + (k / 32) * 4);
}
__device__ __forceinline__ float xt_at(const Lds &L, uint32_t i) { return L.xt[(i & 7u) * L.XT + (i >> 3)]; }
__device__ __forceinline__ void xt_set(const Lds &L, uint32_t i, float v) { L.xt[(i & 7u) * L.XT + (i >> 3)] = v; }

__device__ __forceinline__ void trace_mark(const Cfg &a, uint32_t slot) {
    if (a.trace && threadIdx.x == 0)
        gst(a.trace)[(uint64_t)blockIdx.x * pi_mega_trace_slots(a.n_layer) + slot] = __builtin_amdgcn_s_memrealtime();
}
// Point k (< 32) inside a stage of the middle layer.
__device__ __forceinline__ void trace_detail(const Cfg &a, const Run &r, uint32_t k) {
    if (r.detail) trace_mark(a, 3 + 5 * a.n_layer + k);
}
// Shader-clock counter at point k of the middle layer (with a real-time point
// recorded beside it, two of these give the clock the kernel ran at).
__device__ __forceinline__ void trace_clock(const Cfg &a, const Run &r, uint32_t k) {
    if (r.detail && a.trace && threadIdx.x == 0)
        gst(a.trace)[(uint64_t)blockIdx.x * pi_mega_trace_slots(a.n_layer) + 3 + 5 * a.n_layer + k] =
            __builtin_amdgcn_s_memtime();
}

// ---------------------------------------------------------------------------
// RMSNorm (model.rs:777-823) of the x held in xt, then Q8Act::prepare
// (quant_int.rs:17-56) into L.act.  NEON: simd::f32_sum_sq (simd.rs:45-64):
// eight FMA chains over the stride-8 elements, lane-wise acc0 + acc1, then
// (t0 + t1) + (t2 + t3); else the scalar loop of a multi-token batch.
// out = (x * s) * w.  wr: this thread's 32 norm weights (threads < ne/32).
// ---------------------------------------------------------------------------
struct NoMark {
    __device__ void operator()(uint32_t) const {}
};
// drain = false: loads issued after the input's wait may still be in flight
// (the caller's own tile requests); nothing here waits for them.
template <bool drain = true, typename Mark = NoMark>
__device__ __forceinline__ void norm_q8(const Lds &L, uint32_t ne, float eps, const float4 (&wr)[4], bool neon,
                                        Mark mark = Mark{}) {
    const uint32_t tid = threadIdx.x;
    const uint32_t n4 = ne / 32;  // float4 per transposed row (a multiple of 4: ne % 128 == 0)
    if constexpr (drain) vm_drain();
    mark(12);
    if (neon) {
        if (tid < 8) L.red[tid] = sumsq_fma_chain<6>(reinterpret_cast<const float4 *>(L.xt + tid * L.XT), n4);
        wave_sync();
        if (tid == 0) {
            const float t0 = L.red[0] + L.red[4], t1 = L.red[1] + L.red[5], t2 = L.red[2] + L.red[6],
                        t3 = L.red[3] + L.red[7];
            const float ss = (t0 + t1) + (t2 + t3);
            L.red[8] = 1.0f / sqrtf(ss / (float)ne + eps);
        }
    } else {
        if (tid == 0) {
            float ss = 0.0f;
            for (uint32_t j = 0; j < n4; j++) {
                float4 r[8];
#pragma unroll
                for (int c = 0; c < 8; c++) r[c] = reinterpret_cast<const float4 *>(L.xt + c * L.XT)[j];
#pragma unroll
                for (int q = 0; q < 4; q++)
#pragma unroll
                    for (int c = 0; c < 8; c++) {
                        const float v = comp4(r[c], q);
                        ss += v * v;
                    }
            }
            L.red[8] = 1.0f / sqrtf(ss / (float)ne + eps);
        }
    }
    lds_barrier();
    mark(13);
    const float s = L.red[8];
    if (tid < ne / 16) {
        // elements 16 * tid + j: xt row j % 8, column 2 * tid + j / 8
        const uint32_t b = tid >> 1, h = tid & 1u;
        float v[16];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float2 t = reinterpret_cast<const float2 *>(L.xt + c * L.XT)[tid];
            v[c] = t.x * s * comp4(wr[c / 4], c % 4);
            v[8 + c] = t.y * s * comp4(wr[2 + c / 4], c % 4);
        }
        q8_pair(v, h, L.act.qw + 4 * act_chunk(2 * b + h), L.act.d + b, L.act.s + b);
    }
    lds_barrier();
}

__device__ __forceinline__ void load_norm_w(const float *w, uint32_t ne, float4 (&wr)[4]) {
    if (threadIdx.x < ne / 16) {
        const PI_GLOBAL float4 *w4 = gld(reinterpret_cast<const float4 *>(w + 16 * threadIdx.x));
#pragma unroll
        for (int j = 0; j < 4; j++) wr[j] = w4[j];
    }
}

// Polls n_embd residual words into xt.
__device__ __forceinline__ bool poll_x(const Lds &L, const uint64_t *src, uint32_t ne, uint32_t epoch,
                                       const int32_t *abort_flag) {
    return wg_poll<9>(src, ne, epoch, abort_flag, [&](uint32_t i, uint32_t bits) { xt_set(L, i, __uint_as_float(bits)); });
}

// ---------------------------------------------------------------------------
// GEMV tiles of one matrix set on a Q8 activation in LDS.  A wavefront owns
// tiles first, first + stride, ...; its first P tiles are requested into a
// register ring before the stage waits for its input (prefetch_ring), and
// after tile i is consumed, tile i + P is requested into its slot.
// ---------------------------------------------------------------------------
// Geometry of a matrix set that the tiles of a stage need once the input has
// arrived: total tiles, units per row and this lane's unit within a row.  It
// is read before the wait and passed through an empty asm, so the compiler
// keeps the values in registers instead of re-reading the descriptor (a
// serial chain of scalar-cache misses) after the wait.
struct Geo {
    uint32_t nt, upr, ul, rpw;
};
// A uniform value read from a descriptor, held in registers from here on (see
// Geo).
template <typename V> __device__ __forceinline__ V keep(V v) {
    asm volatile("" : "+s"(v));
    return v;
}
template <typename SS> __device__ __forceinline__ Geo geo_of(const SS &S) {
    Geo g{ms_total(S), ms_upr(S), 0u, ms_rpw(S)};
    g.ul = (threadIdx.x & 63u) % g.upr;
    asm volatile("" : "+s"(g.nt), "+s"(g.upr), "+v"(g.ul), "+s"(g.rpw));
    return g;
}

template <uint32_t T, int G, int P, typename SS>
__device__ __forceinline__ void prefetch_ring(const SS &S, const Geo &g, uint32_t first, uint32_t stride,
                                              Unit<T, G> (&U)[P], TileRef (&R)[P]) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int k = 0; k < P; k++) {
        const uint32_t gt = first + (uint32_t)k * stride;
        if (gt < g.nt) {
            R[k] = tile_ref(S, gt);
            U[k].load(R[k].base, R[k].lanes, min(lane, R[k].lanes - 1));
        }
    }
}

template <uint32_t T, int G, int P, typename SS, typename Out, typename Mark = NoMark>
__device__ __forceinline__ void gemv_ring(const SS &S, const Geo &g, const Lds &L, Unit<T, G> (&U)[P],
                                          TileRef (&R)[P], uint32_t first, uint32_t stride, Out out, Mark mark = Mark{}) {
    const uint32_t lane = threadIdx.x & 63u, nt = g.nt, per_row = g.upr * (QT<T>::TPB * G);
    if (first >= nt) return;
    Slice<T, G> SL;
    SL.load_swz(reinterpret_cast<const int8_t *>(L.act.qw), L.act.d, L.act.s, g.ul);
    mark(29);
    uint32_t gt = first;
    for (;;) {
#pragma unroll
        for (int k = 0; k < P; k++) {
            if (gt >= nt) return;
            consume_tile_pr<T, G>(per_row, SL, U[k], R[k], L.strip, out, mark);
            const uint32_t gn = gt + (uint32_t)P * stride;
            if (gn < nt) {
                R[k] = tile_ref(S, gn);
                U[k].load(R[k].base, R[k].lanes, min(lane, R[k].lanes - 1));
            }
            gt += stride;
        }
    }
}

// One-row tiles (rows longer than 63 units) of a single matrix whose tiles of
// this wavefront are all in the ring (first + P * stride >= total): the terms
// of every tile go to the strip first, then lanes 0..P-1 add their own row's
// terms at once, so the in-order row chains overlap instead of following one
// another.  Row of ring slot k = first + k * stride.
template <uint32_t T, int G, int P, typename SS, typename Out, typename Mark = NoMark>
__device__ __forceinline__ void gemv_ring_rows1(const Geo &g, const Lds &L, const Unit<T, G> (&U)[P],
                                                const TileRef (&R)[P], uint32_t first, uint32_t stride, Out out,
                                                Mark mark = Mark{}) {
    constexpr int TPU = QT<T>::TPB * G;
    const uint32_t lane = threadIdx.x & 63u, per_row = g.upr * TPU;
    if (first >= g.nt) return;
    Slice<T, G> SL;
    SL.load_swz(reinterpret_cast<const int8_t *>(L.act.qw), L.act.d, L.act.s, g.ul);
    uint32_t ntile = 0;
#pragma unroll
    for (int k = 0; k < P; k++) {
        if (first + (uint32_t)k * stride < g.nt) {
            float term[TPU];
            int isum[TPU];
            unit_terms<T, G>(U[k], SL, term, isum);
            if (lane < R[k].lanes) {
#pragma unroll
                for (int t = 0; t < TPU; t++) L.strip[k * per_row + lane * TPU + t] = term[t];
            }
            ntile = (uint32_t)k + 1;
        }
    }
    wave_sync();
    mark(21);
    if (lane < ntile) out(0u, first + lane * stride, 0.0f + chain_sum(L.strip + lane * per_row, per_row));
    wave_sync();
    mark(22);
}

// Calls f(integral_constant<T>, integral_constant<G>) for the runtime type/g.
template <typename F>
__device__ __forceinline__ void with_kq(uint32_t t, F &&f) {
    if (t == PI_TYPE_Q6_K) f(std::integral_constant<uint32_t, PI_TYPE_Q6_K>{}, std::integral_constant<int, 1>{});
    else f(std::integral_constant<uint32_t, PI_TYPE_Q4_K>{}, std::integral_constant<int, 1>{});
}
template <typename F>
__device__ __forceinline__ void with_any(uint32_t t, uint32_t g, F &&f) {
    using I = std::integral_constant<int, 1>;
    switch (t) {
    case PI_TYPE_Q4_K: f(std::integral_constant<uint32_t, PI_TYPE_Q4_K>{}, I{}); return;
    case PI_TYPE_Q6_K: f(std::integral_constant<uint32_t, PI_TYPE_Q6_K>{}, I{}); return;
    default: break;
    }
    auto by_g = [&](auto T) {
        switch (g) {
        case 1: f(T, std::integral_constant<int, 1>{}); return;
        case 2: f(T, std::integral_constant<int, 2>{}); return;
        case 3: f(T, std::integral_constant<int, 3>{}); return;
        case 4: f(T, std::integral_constant<int, 4>{}); return;
        case 6: f(T, std::integral_constant<int, 6>{}); return;
        default: f(T, std::integral_constant<int, 8>{}); return;
        }
    };
    if (t == PI_TYPE_Q4_0) by_g(std::integral_constant<uint32_t, PI_TYPE_Q4_0>{});
    else by_g(std::integral_constant<uint32_t, PI_TYPE_Q8_0>{});
}

#define PI_POLL_OR_LEAVE(expr)                                   \
    do {                                                         \
        if (wg_any(!(expr), L.vote)) {                           \
            if (threadIdx.x == 0) raise_abort(a.abort_flag);     \
            return false;                                        \
        }                                                        \
    } while (0)

// ---------------------------------------------------------------------------
// S1: RMSNorm + Q8 + Q/K/V.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool stage_qkv(const Cfg &a, Run r, const pi_mega_layer *Yp, const Lds &Lc, const uint64_t *xin,
                          uint32_t gw, uint32_t nw) {
    Lds L = Lc;
    set_act_k(L, a.ne);
    bool ok = true;
    const SetRef SA{&Yp->qkv}, SB{&Yp->vb};
    const uint32_t t_qkv = cload(&Yp->t_qkv), t_vb = cload(&Yp->t_vb);
    const float *attn_norm = cload(&Yp->attn_norm);
    uint64_t *oq = keep(cload(&Yp->q)), *okk = keep(cload(&Yp->k)), *ov = keep(cload(&Yp->v));
    const Geo gA = geo_of(SA);
    const Geo gB = ms_n(SB) ? geo_of(SB) : Geo{0u, 1u, 0u, 1u};
    const uint32_t ntA = gA.nt, ntB = gB.nt;
    // segment B continues the wavefront numbering after segment A
    const uint32_t firstB = (gw + nw - ntA % nw) % nw;
    with_kq(t_qkv, [&](auto TA_, auto) {
        with_kq(ntB ? t_vb : t_qkv, [&](auto TB_, auto) {
            constexpr uint32_t TA = decltype(TA_)::value, TB = decltype(TB_)::value;
            Unit<TA, 1> UA[1];
            Unit<TB, 1> UB[1];
            TileRef RA[1], RB[1];
            const bool b_first = gw >= ntA && firstB < ntB;   // B is this wavefront's first work
            // The first tile is requested in two halves: the first before the
            // wait for the residual, the second once it has arrived (the
            // wait's loads complete only after every load issued before them,
            // and the norm that follows takes longer than the second half).
            const uint32_t lane = threadIdx.x & 63u;
            constexpr int HA = Unit<TA, 1>::QC / 2, HB = Unit<TB, 1>::QC / 2;
            const bool has = b_first || gw < ntA;
            if (b_first) RB[0] = tile_ref(SB, firstB);
            else if (gw < ntA) RA[0] = tile_ref(SA, gw);
            if (b_first) UB[0].template load_part<0, HB>(RB[0].base, RB[0].lanes, min(lane, RB[0].lanes - 1));
            else if (has) UA[0].template load_part<0, HA>(RA[0].base, RA[0].lanes, min(lane, RA[0].lanes - 1));
            lds_barrier();
            if (xin) ok = poll_x(L, xin, a.ne, r.epoch, a.abort_flag);
            if (wg_any(!ok, L.vote)) { ok = false; return; }
            trace_detail(a, r, 0);
            float4 wr[4];   // needed only after the sum of squares: requested after the wait too
            load_norm_w(attn_norm, a.ne, wr);
            // (clock point 14 used by the attention trace)
            if (b_first)
                UB[0].template load_part<HB, Unit<TB, 1>::QC>(RB[0].base, RB[0].lanes, min(lane, RB[0].lanes - 1));
            else if (has)
                UA[0].template load_part<HA, Unit<TA, 1>::QC>(RA[0].base, RA[0].lanes, min(lane, RA[0].lanes - 1));
            norm_q8<false>(L, a.ne, a.eps, wr, r.neon, [&](uint32_t k) { trace_detail(a, r, k); });
            trace_detail(a, r, 1);
            auto outA = [&](uint32_t m, uint32_t row, float v) {
                uint64_t *o = m == 0 ? oq : (m == 1 ? okk : ov);
                ll_put(o + row, __float_as_uint(v), r.epoch);
            };
            auto outB = [&](uint32_t, uint32_t row, float v) { ll_put(ov + row, __float_as_uint(v), r.epoch); };
            if (b_first) {
                gemv_ring<TB, 1, 1>(SB, gB, L, UB, RB, firstB, nw, outB);
            } else {
                gemv_ring<TA, 1, 1>(SA, gA, L, UA, RA, gw, nw, outA);
                if (firstB < ntB) {
                    prefetch_ring<TB, 1, 1>(SB, gB, firstB, nw, UB, RB);
                    gemv_ring<TB, 1, 1>(SB, gB, L, UB, RB, firstB, nw, outB);
                }
            }
            trace_detail(a, r, 2);
        });
    });
    if (!ok && threadIdx.x == 0) raise_abort(a.abort_flag);
    return ok;
}

// ---------------------------------------------------------------------------
// S2: attention of head h for the token at r.pos (model.rs:953-1087).
// RoPE of q and k over adjacent pairs, K/V row write (first head of a KV
// group), scores q.k_p * scale for p = 0..pos (NEON: simd::f32_dot's two
// 4-lane accumulators; else the scalar loop), max, e_p = exp(s_p - max),
// sum over p in order, o[d] = sum over p in order of e_p * v_p[d] skipping
// e_p == 0 (f32_axpy: product rounded, then added), o * (1/sum), Q8 of o.
// Two workgroups per head (seg 0 and 1) each form o for one half of the
// dimensions, which is also one Q8 block of the output; at long contexts
// more workgroups take segments of the scores.  In a chain workgroup,
// wavefronts 1-3 form the products of the next chunk of positions while
// wavefront 0 adds the current chunk in order (lane = dimension) and, in its
// upper lanes, the running sum of e_p.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool stage_attn(const Cfg &a, Run r, const pi_mega_layer *Yp, const Lds &L, uint32_t h,
                                           uint32_t seg, uint32_t nseg, uint32_t layer) {
    constexpr uint32_t DH = 64;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t group = a.n_head / a.n_kv, kvh = h / group;
    const int pos = r.pos;
    const uint32_t n = (uint32_t)pos + 1;
    // positions [p0, p1) of this workgroup's scores: every position when the
    // head has a single score segment (both chain workgroups score it all),
    // else segment seg of nseg
    const uint32_t p0 = nseg == 1 ? 0u : (uint32_t)((uint64_t)seg * n / nseg);
    const uint32_t p1 = nseg == 1 ? n : (uint32_t)((uint64_t)(seg + 1) * n / nseg);
    const uint32_t tag = r.epoch * 64u + layer + 1u;
    const uint64_t *yq = cload(&Yp->q), *yk = cload(&Yp->k), *yv = cload(&Yp->v);
    uint64_t *yatt = cload(&Yp->att);
    float *ykc = cload(&Yp->kc), *yvc = cload(&Yp->vc);
    float *qs = L.red, *kcur = L.red + 64, *vcur = L.red + 128, *misc = L.red + 192;
    float *kbase = ykc + (uint64_t)kvh * a.n_ctx * DH;
    float *vbase = yvc + (uint64_t)kvh * a.n_ctx * DH;
    // Every K row is requested from HBM (the row of the current position may
    // not be visible yet; the score loop takes it from LDS), so loads never share a
    // destination register with an LDS read.
    auto load_k = [&](uint32_t p, float4 (&kr)[16]) {
        const PI_GLOBAL float4 *src = gld(reinterpret_cast<const float4 *>(kbase + (uint64_t)p * DH));
#pragma unroll
        for (int i = 0; i < 16; i++) kr[i] = src[i];
    };
    // the first K row of this thread is requested before the inputs arrive
    float4 kr[16];
    if (p0 + tid < p1) load_k(p0 + tid, kr);
    // inputs: q of head h, k and v of its KV head
    bool ok = true;
    if (tid < 3 * DH) {
        const uint32_t part = tid / DH, d = tid % DH;
        const uint64_t *src = part == 0 ? yq + h * DH + d : (part == 1 ? yk + kvh * DH + d : yv + kvh * DH + d);
        uint64_t w = ll_get(src);
        ok = ll_wait(src, r.epoch, w, a.abort_flag);
        L.red[tid] = __uint_as_float((uint32_t)w);
    }
    PI_POLL_OR_LEAVE(ok);
    trace_detail(a, r, 3);
    const PI_GLOBAL float *cb = gld(a.cos_tab + (uint64_t)pos * a.half), *sb = gld(a.sin_tab + (uint64_t)pos * a.half);
    if (tid < DH / 2 && tid < a.half) {
        const uint32_t i = tid;
        const float c = cb[i], s = sb[i];
        const float x0 = qs[2 * i], x1 = qs[2 * i + 1], y0 = kcur[2 * i], y1 = kcur[2 * i + 1];
        qs[2 * i] = x0 * c - x1 * s;
        qs[2 * i + 1] = x0 * s + x1 * c;
        kcur[2 * i] = y0 * c - y1 * s;
        kcur[2 * i + 1] = y0 * s + y1 * c;
    }
    lds_barrier();
    trace_detail(a, r, 20);
    if (seg == 0 && h % group == 0 && tid < DH) {
        gst(kbase)[(uint64_t)pos * DH + tid] = kcur[tid];
        gst(vbase)[(uint64_t)pos * DH + tid] = vcur[tid];
    }
    // scores; the K row of the next position of this thread is requested
    // before the current one is used
    float mx = -INFINITY;
    const float4 *q4 = reinterpret_cast<const float4 *>(qs);
    auto score = [&](const float4 (&kr)[16]) {
        float s;
        if (r.neon) {
            float a0[4] = {0.f, 0.f, 0.f, 0.f}, a1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 qa = q4[2 * i], qb = q4[2 * i + 1], ka = kr[2 * i], kb = kr[2 * i + 1];
                a0[0] = a0[0] + qa.x * ka.x; a0[1] = a0[1] + qa.y * ka.y;
                a0[2] = a0[2] + qa.z * ka.z; a0[3] = a0[3] + qa.w * ka.w;
                a1[0] = a1[0] + qb.x * kb.x; a1[1] = a1[1] + qb.y * kb.y;
                a1[2] = a1[2] + qb.z * kb.z; a1[3] = a1[3] + qb.w * kb.w;
            }
            s = (a0[0] + a0[1]) + (a0[2] + a0[3]);
            s += (a1[0] + a1[1]) + (a1[2] + a1[3]);
        } else {
            s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float4 qa = q4[i], ka = kr[i];
                s += qa.x * ka.x;
                s += qa.y * ka.y;
                s += qa.z * ka.z;
                s += qa.w * ka.w;
            }
        }
        return s * a.scale;
    };
    for (uint32_t p = p0 + tid; p < p1; p += MT) {
        float4 kn[16];
        if (p + MT < p1) load_k(p + MT, kn);
        if (p == (uint32_t)pos) {   // this position's row: from LDS
#pragma unroll
            for (int i = 0; i < 16; i++) kr[i] = reinterpret_cast<const float4 *>(kcur)[i];
        }
        const float s = score(kr);
        L.sc[p] = s;
        mx = fmaxf(mx, s);
#pragma unroll
        for (int i = 0; i < 16; i++) kr[i] = kn[i];
    }
    trace_detail(a, r, 28);
    vm_drain();
    // The value chain of this head is split by dimension: workgroups 0 and 1
    // of the head each add dimensions 32 * half .. + 31 (half = seg), which is
    // also the split of the output into its two Q8 blocks.
    constexpr uint32_t DHH = DH / 2;
    constexpr int GPW = 3;        // 8 groups of 8 positions per chunk over 3 product wavefronts
    constexpr int kDepth = 4;
    const uint32_t half = seg;
    const uint32_t nchunk = (n + kChunk - 1) / kChunk;
    const uint32_t dl = 4 * (lane & 7u), sub = lane >> 3;   // dimensions dl..dl+3 of the half, position 8g + sub
    const float4 vme = reinterpret_cast<const float4 *>(vcur + DHH * (half & 1u))[lane & 7u];
    float4 vr[kDepth][GPW];
    auto load_v = [&](uint32_t c, float4 (&v)[GPW]) {
#pragma unroll
        for (int i = 0; i < GPW; i++) {
            const uint32_t g = (wave - 1) + (MW - 1) * i;
            const uint32_t p = min(c * kChunk + 8 * g + sub, n - 1);
            v[i] = gld(reinterpret_cast<const float4 *>(vbase + (uint64_t)p * DH + DHH * half))[lane & 7u];
        }
    };
    // the chain workgroups request their first V rows before the softmax
    // (unconditionally: load_v clamps to row n - 1, and a fixed number of
    // loads per ring slot lets the compiler wait for the oldest slot only)
    if (seg < 2 && wave != 0) {
#pragma unroll
        for (int k = 0; k < kDepth; k++) load_v(k, vr[k]);
    }
    trace_detail(a, r, 15);
    mx = wave_max(mx);
    if (lane == 0) misc[wave] = mx;
    lds_barrier();
    mx = fmaxf(fmaxf(misc[0], misc[1]), fmaxf(misc[2], misc[3]));
    if (nseg > 1) {
        // maximum over every segment of the head (exact in any order)
        uint64_t *am = a.amax + (uint64_t)h * PI_MEGA_MAX_SEG;
        if (tid == 0) ll_put(am + seg, __float_as_uint(mx), tag);
        bool okm = true;
        if (tid < nseg) {
            uint64_t wv = ll_get(am + tid);
            okm = ll_wait(am + tid, tag, wv, a.abort_flag);
            misc[8 + tid] = __uint_as_float((uint32_t)wv);
        }
        PI_POLL_OR_LEAVE(okm);
        for (uint32_t i = 0; i < nseg; i++) mx = fmaxf(mx, misc[8 + i]);
    }
    for (uint32_t p = p0 + tid; p < p1; p += MT) L.sc[p] = pi_expf(L.sc[p] - mx);
    trace_detail(a, r, 14);
    if (nseg > 1) {
        // every segment publishes its e_p; the two chain workgroups read the
        // positions outside their own segment
        uint64_t *ae = a.aexp + (uint64_t)h * a.n_ctx;
        for (uint32_t p = p0 + tid; p < p1; p += MT) ll_put(ae + p, __float_as_uint(L.sc[p]), tag);
        if (seg >= 2) {
            lds_barrier();
            return true;
        }
        bool oke = wg_poll<8>(ae, p0, tag, a.abort_flag, [&](uint32_t i, uint32_t bits) { L.sc[i] = __uint_as_float(bits); });
        if (oke)
            oke = wg_poll<8>(ae + p1, n - p1, tag, a.abort_flag,
                             [&](uint32_t i, uint32_t bits) { L.sc[p1 + i] = __uint_as_float(bits); });
        PI_POLL_OR_LEAVE(oke);
    }
    // e_p = 0 past the last position up to the end of its chunk, so every
    // chunk is added whole: both sums start at +0 and never become -0, so
    // adding +0 leaves them unchanged.
    for (uint32_t p = n + tid; p < nchunk * kChunk; p += MT) L.sc[p] = 0.0f;
    lds_barrier();
    trace_detail(a, r, 4);

    // Products e_p * v_p[d] of chunk c go to buffer c & 1: row d of the half
    // (32 rows), float4 group (p / 4) ^ ((d / 8) & 3), row pitch kChunkPad.
    // The pitch and the group permutation keep the producers' single-float
    // stores (4 dimensions x 8 positions per 32 lanes) and the adder's float4
    // reads (one row per lane) on distinct banks.  Wavefronts 1-3 own groups
    // w-1, w+2, ... of 8 positions (lane l: position 8g + l/8, dimensions
    // dl..dl+3, one 16-byte load) and keep the V rows of the next kDepth
    // chunks in flight in registers.  V rows always come from HBM (rows past
    // the end re-read row n-1, whose product is 0 since e_p = 0 there); the
    // current position's row is taken from LDS.  e_p == 0 skips the position
    // (f32_axpy), which only matters for a non-finite v: a chunk with no zero
    // weight, away from the current position, takes the plain products (the
    // vote is uniform per wavefront).
    const uint32_t cpos = (uint32_t)pos / kChunk;
    auto store_products = [&](uint32_t c, const float4 (&v)[GPW]) {
        float *buf = L.hb + (c & 1u) * DHH * kChunkPad + dl * kChunkPad;
        const uint32_t hq = (lane & 7u) >> 1;   // (d / 8) & 3 for d = dl .. dl + 3
        float e[GPW];
        bool anyz = false;
#pragma unroll
        for (int i = 0; i < GPW; i++) {   // all weights first, so their reads overlap
            const uint32_t g = (wave - 1) + (MW - 1) * i;
            e[i] = L.sc[c * kChunk + min(8 * g + sub, kChunk - 1)];
            anyz |= e[i] == 0.0f;
        }
        if (!__builtin_amdgcn_readfirstlane(__ballot(anyz) != 0 || c == cpos)) {
#pragma unroll
            for (int i = 0; i < GPW; i++) {
                const uint32_t g = (wave - 1) + (MW - 1) * i;
                if (g < kChunk / 8) {
                    const uint32_t col = 4 * ((2 * g + (sub >> 2)) ^ hq) + (sub & 3u);
                    buf[0 * kChunkPad + col] = e[i] * v[i].x;
                    buf[1 * kChunkPad + col] = e[i] * v[i].y;
                    buf[2 * kChunkPad + col] = e[i] * v[i].z;
                    buf[3 * kChunkPad + col] = e[i] * v[i].w;
                }
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < GPW; i++) {
            const uint32_t g = (wave - 1) + (MW - 1) * i;
            if (g < kChunk / 8) {
                const uint32_t p = c * kChunk + 8 * g + sub;
                const uint32_t col = 4 * ((2 * g + (sub >> 2)) ^ hq) + (sub & 3u);
                const float4 vv = p == (uint32_t)pos ? vme : v[i];
                const bool nz = e[i] != 0.0f;
                buf[0 * kChunkPad + col] = nz ? e[i] * vv.x : 0.0f;
                buf[1 * kChunkPad + col] = nz ? e[i] * vv.y : 0.0f;
                buf[2 * kChunkPad + col] = nz ? e[i] * vv.z : 0.0f;
                buf[3 * kChunkPad + col] = nz ? e[i] * vv.w : 0.0f;
            }
        }
    };
    // Step c (0..nchunk): wavefronts 1-3 store the products of chunk c and
    // refill the ring slot they used with the rows of chunk c + kDepth;
    // wavefront 0 adds chunk c - 1: lanes 0-31 their dimension's products,
    // lanes 32-63 the weights (the sum of e_p, the same in each of them), so
    // one add per position covers both chains.  Producers and adder run
    // separate loops with the same barrier count.  In the producers' main
    // loop every step of a group issues the same loads, so each ring slot
    // keeps its own registers and a wavefront waits only for its oldest slot
    // while the others stay in flight; the last steps, whose rows are already
    // requested, run without refills.
    float acc = 0.0f;
    if (wave != 0) {
        uint32_t c0 = 0;
        for (; c0 + kDepth <= nchunk; c0 += kDepth) {
#pragma unroll
            for (int k = 0; k < kDepth; k++) {
                const uint32_t c = c0 + k;
                store_products(c, vr[k]);
                load_v(c + kDepth, vr[k]);
                lds_barrier();
            }
        }
#pragma unroll
        for (int k = 0; k < kDepth; k++) {   // steps c0 .. nchunk (at most kDepth of them)
            const uint32_t c = c0 + k;
            if (c > nchunk) continue;   // uniform over the workgroup
            if (c < nchunk) store_products(c, vr[k]);
            lds_barrier();
        }
    } else {
        const bool wlane = lane >= DHH;                          // weight lanes
        const uint32_t hr = wlane ? 0u : (lane >> 3) & 3u;       // (d / 8) & 3 of this lane's row
        // The lane's row base is fixed and the step's offset is formed with a
        // mask, so the loop runs without divergent branches (a select
        // between the two rows compiles to an exec-masked branch per step).
        const float *base = wlane ? L.sc : L.hb + lane * kChunkPad;
        const uint32_t ncu = __builtin_amdgcn_readfirstlane(nchunk);
        const uint32_t wmask = wlane ? ~0u : 0u;
        for (uint32_t c = 0; c <= ncu; c++) {
            if (c >= 1) {
                const uint32_t off = ((c - 1) * kChunk & wmask) | (((c - 1) & 1u) * DHH * kChunkPad & ~wmask);
                const float4 *src = reinterpret_cast<const float4 *>(base + off);
                // all 16 reads of the chunk first (the scheduling barrier keeps
                // them ahead of the adds), one LDS latency per step
                float4 t[16];
#pragma unroll
                for (int q = 0; q < 16; q++) t[q] = src[q ^ hr];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    acc = acc + t[q].x;
                    acc = acc + t[q].y;
                    acc = acc + t[q].z;
                    acc = acc + t[q].w;
                }
            }
            lds_barrier();
        }
    }
    trace_detail(a, r, 5);
    if (wave == 0) {
        const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), DHH));   // sum of e_p
        const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
        const float o = acc * inv;                               // lanes 0-31: this half's outputs
        float dd;
        int bs;
        const int iv = q8_block32_core(o, dd, bs);               // lanes 32-63 form a block that is not used
        int8_t *qst = reinterpret_cast<int8_t *>(misc + 16);     // 32 quants
        if (lane < DHH) qst[lane] = (int8_t)iv;
        wave_sync();
        // att words: quants (16 per head, 8 per half), then qdim/32 scales, then qdim/32 sums
        const uint32_t qdim = a.n_head * DH;
        if (lane < 8) ll_put(yatt + h * 16 + half * 8 + lane, reinterpret_cast<const uint32_t *>(qst)[lane], r.epoch);
        else if (lane == 8) ll_put(yatt + qdim / 4 + h * 2 + half, __float_as_uint(dd), r.epoch);
        else if (lane == 9) ll_put(yatt + qdim / 4 + qdim / 32 + h * 2 + half, (uint32_t)bs, r.epoch);
    }
    trace_detail(a, r, 16);
    lds_barrier();
    trace_detail(a, r, 17);
    return true;
}

// ---------------------------------------------------------------------------
// h blocks of the gate/up stage (S4).
// ---------------------------------------------------------------------------
// Block mode (h_q8): the workgroup of block b (h_first_block, then b +
// gridDim.x, ...) evaluates rows 32b .. 32b + 31 of gate and of up, forms that
// Q8 block of h and publishes it
// quantized (Q8Act::prepare, quant_int.rs:17-56): 8 quant words, d and the
// block sum, so ffn_down reads 10 words per block instead of 32 floats and
// quantizes nothing.  Wavefront w takes rows 32b + 8w + i (i < 8) of gate
// (row-dots i) and of up (row-dots 8 + i).  Lane s * upr + j (slot s < rpw)
// holds unit j of row-dots s, s + rpw, s + 2 rpw, so it keeps the activation
// slice of one column; lanes past rpw * upr idle.  Each row-dot's terms go to
// the wavefront's strip in the h staging area, then lanes 0..15 add their
// row-dot's terms in order at the same time (gate in lanes 0..7, up in 8..15).
constexpr int kHU = 3;           // units per lane
constexpr uint32_t kHRowDots = 16;

__host__ __device__ inline uint32_t h_strip_floats(uint32_t upr, uint32_t tpu) {
    return (kHRowDots * upr * tpu + kChainPad + 3u) & ~3u;
}

template <uint32_t T>
__device__ __forceinline__ void h_units(const SetRef &S, const Geo &g, uint32_t n_ff, uint32_t b,
                                        Unit<T, 1> (&U)[kHU]) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = lane / g.upr;
    const uint32_t ntl = ms_t0(S, 1), lpt = ms_lpt(S);
    const uint64_t tb = ms_tb(S);
    const uint8_t *wg = ms_w(S, 0), *wu = ms_w(S, 1);
#pragma unroll
    for (int k = 0; k < kHU; k++) {
        const uint32_t rd = slot + (uint32_t)k * g.rpw;
        if (slot < g.rpw && rd < kHRowDots) {
            const uint32_t row = 32u * b + 8u * wave + (rd & 7u);
            const uint32_t t = row / g.rpw, lr = row - t * g.rpw;
            const uint32_t lanes = t == ntl - 1 ? (n_ff - t * g.rpw) * g.upr : lpt;
            U[k].load((rd < 8 ? wg : wu) + (uint64_t)t * tb, lanes, lr * g.upr + g.ul);
        }
    }
}

template <uint32_t T>
__device__ __forceinline__ void h_block(const Cfg &a, const Run &r, const SetRef &S, const Geo &g, const Lds &L,
                                        const Slice<T, 1> &SL, const Unit<T, 1> (&U)[kHU], uint32_t b, uint64_t *yh) {
    constexpr int TPU = QT<T>::TPB;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t slot = lane / g.upr, per_row = g.upr * TPU;
    float *strip = L.hb + wave * h_strip_floats(g.upr, TPU);
#pragma unroll
    for (int k = 0; k < kHU; k++) {
        const uint32_t rd = slot + (uint32_t)k * g.rpw;
        if (slot < g.rpw && rd < kHRowDots) {
            float term[TPU];
            int isum[TPU];
            unit_terms<T, 1>(U[k], SL, term, isum);
#pragma unroll
            for (int t = 0; t < TPU; t++) strip[rd * per_row + g.ul * TPU + t] = term[t];
        }
    }
    wave_sync();
    trace_detail(a, r, 24);
    float v = 0.0f;
    if (lane < kHRowDots) v = 0.0f + chain_sum(strip + lane * per_row, per_row);
    const float u = dpp<0x128>(v);   // row_ror:8: lane i < 8 receives up row-dot i from lane i + 8
    float *hv = L.red + 32;          // h of rows 32b .. 32b + 31
    if (lane < 8) {
        const float sg = v / (1.0f + pi_expf(-v));
        hv[8 * wave + lane] = sg * u;
    }
    trace_detail(a, r, 25);
    lds_barrier();
    trace_detail(a, r, 26);
    if (wave == 0) {
        float dd;
        int bs;
        const int iv = q8_block32_core(lane < 32 ? hv[lane] : 0.0f, dd, bs);   // lanes 32-63: a block not used
        int8_t *qst = reinterpret_cast<int8_t *>(L.red + 64);
        if (lane < 32) qst[lane] = (int8_t)iv;
        wave_sync();
        const uint32_t nq = a.n_ff / 4;
        if (lane < 8) ll_put(yh + 8 * b + lane, reinterpret_cast<const uint32_t *>(qst)[lane], r.epoch);
        else if (lane == 8) ll_put(yh + nq + b, __float_as_uint(dd), r.epoch);
        else if (lane == 9) ll_put(yh + nq + a.n_ff / 32 + b, (uint32_t)bs, r.epoch);
    }
    trace_detail(a, r, 27);
    lds_barrier();   // hv, the quants and the strips are free for the next block
}

// The block mode's gate/up units of this workgroup's first block (Q4_K).
using HUnits = Unit<PI_TYPE_Q4_K, 1>[kHU];
// Marks the units' previous contents as dead (no instruction): without it the
// conditional loads below would keep the last layer's units live around the
// whole layer loop.
__device__ __forceinline__ void h_units_fresh(HUnits &U) {
#pragma unroll
    for (int k = 0; k < kHU; k++)
#pragma unroll
        for (int j = 0; j < Unit<PI_TYPE_Q4_K, 1>::QC; j++)
            asm volatile("" : "=v"(U[k].c[j].x), "=v"(U[k].c[j].y), "=v"(U[k].c[j].z), "=v"(U[k].c[j].w));
}
// First h block of this workgroup: blocks are numbered from the last
// workgroup down, away from the first workgroups, which hold the attn_output
// tiles.
__device__ __forceinline__ uint32_t h_first_block() { return gridDim.x - 1 - blockIdx.x; }

// ---------------------------------------------------------------------------
// S3: attn_output on the attention's Q8, x + proj -> xb (model.rs:1091-1097).
// ---------------------------------------------------------------------------
// HU / hpre: see stage_ffn_up.  early: the workgroup ran no attention in this
// layer, so it gets here while attention is still running.
__device__ __forceinline__ bool stage_o(const Cfg &a, Run r, const pi_mega_layer *Yp, const Lds &Lc, uint32_t gw, uint32_t nw,
                                        HUnits &HU, bool &hpre, bool early) {
    Lds L = Lc;
    const uint32_t qdim = a.n_head * 64;
    set_act_k(L, qdim);
    bool ok = true;
    const SetRef SO{&Yp->o};
    const uint32_t t_o = cload(&Yp->t_o), g_o = cload(&Yp->g_o);
    const uint64_t *yatt = cload(&Yp->att);
    uint64_t *yxb = keep(cload(&Yp->xb));
    with_any(t_o, g_o, [&](auto T_, auto G_) {
        constexpr uint32_t T = decltype(T_)::value;
        constexpr int G = decltype(G_)::value;
        Unit<T, G> U[1];
        TileRef R[1];
        const Geo g = geo_of(SO);
        if (blockIdx.x * MW >= g.nt) return;   // no tile in this workgroup: nothing to wait for
        prefetch_ring<T, G, 1>(SO, g, gw, nw, U, R);
        if constexpr (T == PI_TYPE_Q4_K) {   // (the other types leave too few registers)
            if (cload(&Yp->h_q8) && h_first_block() < a.n_ff / 32) {
                // this workgroup also evaluates an h block: its gate/up units
                // are requested now, long before the residual they need arrives
                const SetRef SGU{&Yp->gu};
                h_units<PI_TYPE_Q4_K>(SGU, geo_of(SGU), a.n_ff, h_first_block(), HU);
                hpre = true;
            }
        }
        lds_barrier();
        if (early) __builtin_amdgcn_s_sleep(127);   // poll later: less traffic for the polls that matter
        const uint32_t nwords = qdim / 4 + qdim / 16, nq = qdim / 4;
        ok = wg_poll<3>(yatt, nwords, r.epoch, a.abort_flag, [&](uint32_t i, uint32_t bits) {
            L.act.qw[i < nq ? 4 * act_chunk(i >> 2) + (i & 3u) : i] = bits;
        });
        if (wg_any(!ok, L.vote)) { ok = false; return; }
        trace_detail(a, r, 18);
        auto out = [&](uint32_t, uint32_t row, float v) {
            ll_put(yxb + row, __float_as_uint(xt_at(L, row) + v), r.epoch);
        };
        gemv_ring<T, G, 1>(SO, g, L, U, R, gw, nw, out, [&](uint32_t k) { trace_detail(a, r, k); });
        trace_detail(a, r, 19);
    });
    if (!ok && threadIdx.x == 0) raise_abort(a.abort_flag);
    return ok;
}

// ---------------------------------------------------------------------------
// S4: RMSNorm + Q8 of xb, gate/up tile pairs, h = silu(gate) * up
// (model.rs:1099-1115).
// ---------------------------------------------------------------------------
// hpre: the units of the first block were requested during the attn_output
// stage (workgroups that also hold an attn_output tile).
// early: the workgroup ran neither attention nor an attn_output tile in this
// layer, so it reaches this stage long before the residual exists.
__device__ __forceinline__ bool stage_ffn_up(const Cfg &a, Run r, const pi_mega_layer *Yp, const Lds &Lc, uint32_t gw,
                                             uint32_t nw, HUnits &HU, bool hpre, bool early) {
    Lds L = Lc;
    set_act_k(L, a.ne);
    bool ok = true;
    const SetRef SGU{&Yp->gu};
    const uint32_t t_gu = cload(&Yp->t_gu);
    const float *ffn_norm = cload(&Yp->ffn_norm);
    const uint64_t *yxb = cload(&Yp->xb);
    uint64_t *yh = keep(cload(&Yp->h));
    if (cload(&Yp->h_q8)) {
        constexpr uint32_t T = PI_TYPE_Q4_K;
        const Geo g = geo_of(SGU);
        const uint32_t nblk = a.n_ff / 32, nb = gridDim.x, b0 = h_first_block();
        if (b0 < nblk && !hpre) h_units<T>(SGU, g, a.n_ff, b0, HU);
        float4 wr[4];
        load_norm_w(ffn_norm, a.ne, wr);
        lds_barrier();
        // Without an h block the residual is needed only by ffn_down, and a
        // workgroup that skipped attention and attn_output waits the better
        // part of those two stages: both poll later, so the polls that matter
        // see less traffic.
        if (b0 >= nblk) __builtin_amdgcn_s_sleep(64);
        else if (early) {
            __builtin_amdgcn_s_sleep(127);
            __builtin_amdgcn_s_sleep(127);
        }
        ok = poll_x(L, yxb, a.ne, r.epoch, a.abort_flag);
        PI_POLL_OR_LEAVE(ok);
        trace_detail(a, r, 6);
        norm_q8(L, a.ne, a.eps, wr, r.neon);
        trace_detail(a, r, 7);
        if (b0 >= nblk) return true;
        Slice<T, 1> SL;
        SL.load_swz(reinterpret_cast<const int8_t *>(L.act.qw), L.act.d, L.act.s, g.ul);
        for (uint32_t b = b0; b < nblk; b += nb) {
            if (b != b0) h_units<T>(SGU, g, a.n_ff, b, HU);
            h_block<T>(a, r, SGU, g, L, SL, HU, b, yh);
        }
        trace_detail(a, r, 8);
        return true;
    }
    with_kq(t_gu, [&](auto T_, auto) {
        constexpr uint32_t T = decltype(T_)::value;
        constexpr int TPU = QT<T>::TPB;
        const uint32_t lane = threadIdx.x & 63u;
        const SetRef &S = SGU;
        const Geo g = geo_of(S);
        const uint32_t npair = ms_t0(S, 1);
        const uint32_t p0 = gw;
        Unit<T, 1> Ug, Uu;
        TileRef Rg{}, Ru{};
        if (gw < npair) {
            Rg = tile_ref(S, p0);
            Ru = tile_ref(S, npair + p0);
            Ug.load(Rg.base, Rg.lanes, min(lane, Rg.lanes - 1));
            Uu.load(Ru.base, Ru.lanes, min(lane, Ru.lanes - 1));
        }
        float4 wr[4];
        load_norm_w(ffn_norm, a.ne, wr);
        lds_barrier();
        ok = poll_x(L, yxb, a.ne, r.epoch, a.abort_flag);
        if (wg_any(!ok, L.vote)) { ok = false; return; }
        trace_detail(a, r, 6);
        norm_q8(L, a.ne, a.eps, wr, r.neon);
        trace_detail(a, r, 7);
        if (gw >= npair) return;
        Slice<T, 1> SL;
        SL.load_swz(reinterpret_cast<const int8_t *>(L.act.qw), L.act.d, L.act.s, g.ul);
        const uint32_t per_row = g.upr * TPU;
        for (uint32_t p = gw; p < npair; p += nw) {
            if (p != p0) {
                Rg = tile_ref(S, p);
                Ru = tile_ref(S, npair + p);
                Ug.load(Rg.base, Rg.lanes, min(lane, Rg.lanes - 1));
                Uu.load(Ru.base, Ru.lanes, min(lane, Ru.lanes - 1));
            }
            float term[TPU];
            int isum[TPU];
            unit_terms<T, 1>(Ug, SL, term, isum);
            if (lane < Rg.lanes) {
#pragma unroll
                for (int t = 0; t < TPU; t++) L.strip[lane * TPU + t] = term[t];
            }
            wave_sync();
            float g = 0.0f;
            if (lane < Rg.nrows) g = 0.0f + chain_sum(L.strip + lane * per_row, per_row);
            wave_sync();
            trace_detail(a, r, 20);
            unit_terms<T, 1>(Uu, SL, term, isum);
            if (lane < Ru.lanes) {
#pragma unroll
                for (int t = 0; t < TPU; t++) L.strip[lane * TPU + t] = term[t];
            }
            wave_sync();
            if (lane < Ru.nrows) {
                const float u = 0.0f + chain_sum(L.strip + lane * per_row, per_row);
                const float sg = g / (1.0f + pi_expf(-g));
                ll_put(yh + Rg.row0 + lane, __float_as_uint(sg * u), r.epoch);
            }
            wave_sync();
        }
        trace_detail(a, r, 8);
    });
    if (!ok && threadIdx.x == 0) raise_abort(a.abort_flag);
    return ok;
}

// ---------------------------------------------------------------------------
// S5: Q8 of h, ffn_down, xb + proj -> xo (model.rs:1119-1125).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool stage_down(const Cfg &a, Run r, const pi_mega_layer *Yp, const Lds &Lc, uint32_t gw, uint32_t nw) {
    Lds L = Lc;
    set_act_k(L, a.n_ff);
    bool ok = true;
    const SetRef SD{&Yp->down};
    const uint32_t t_down = cload(&Yp->t_down), g_down = cload(&Yp->g_down);
    const uint64_t *yh = cload(&Yp->h);
    const uint32_t hq8 = cload(&Yp->h_q8);
    uint64_t *yxo = keep(cload(&Yp->xo));
    with_any(t_down, g_down, [&](auto T_, auto G_) {
        constexpr uint32_t T = decltype(T_)::value;
        constexpr int G = decltype(G_)::value;
        Unit<T, G> U[3];
        TileRef R[3];
        const Geo g = geo_of(SD);
        prefetch_ring<T, G, 3>(SD, g, gw, nw, U, R);
        lds_barrier();
        if (hq8) {
            // Q8 blocks of h as the gate/up stage published them
            const uint32_t nq = a.n_ff / 4;
            ok = wg_poll<8>(yh, nq + a.n_ff / 16, r.epoch, a.abort_flag, [&](uint32_t i, uint32_t bits) {
                L.act.qw[i < nq ? 4 * act_chunk(i >> 2) + (i & 3u) : i] = bits;
            });
            if (wg_any(!ok, L.vote)) { ok = false; return; }
            trace_detail(a, r, 9);
        } else {
        ok = wg_poll<23>(yh, a.n_ff, r.epoch, a.abort_flag,
                         [&](uint32_t i, uint32_t bits) { L.hb[i] = __uint_as_float(bits); });
        if (wg_any(!ok, L.vote)) { ok = false; return; }
        trace_detail(a, r, 9);
        for (uint32_t t = threadIdx.x; t < a.n_ff / 16; t += MT) {   // pairs of lanes stay together
            const uint32_t b = t >> 1, h = t & 1u;
            float v[16];
            const float4 *x4 = reinterpret_cast<const float4 *>(L.hb + 16 * t);
#pragma unroll
            for (int j4 = 0; j4 < 4; j4++) {
                const float4 q = x4[j4];
                v[4 * j4 + 0] = q.x;
                v[4 * j4 + 1] = q.y;
                v[4 * j4 + 2] = q.z;
                v[4 * j4 + 3] = q.w;
            }
            q8_pair(v, h, L.act.qw + 4 * act_chunk(2 * b + h), L.act.d + b, L.act.s + b);
        }
        lds_barrier();
        }
        trace_detail(a, r, 10);
        auto out = [&](uint32_t, uint32_t row, float v) {
            ll_put(yxo + row, __float_as_uint(xt_at(L, row) + v), r.epoch);
        };
        if constexpr (T == PI_TYPE_Q4_0 || T == PI_TYPE_Q8_0) {
            constexpr uint32_t TPU = QT<T>::TPB * G;
            // every tile of this wavefront in the ring, and three rows of terms
            // (plus the chain reader's read-ahead) inside its strip
            if (g.rpw == 1 && ms_n(SD) == 1 && gw + 3 * nw >= g.nt && 3 * g.upr * TPU + kChainPad <= 64u * 16u) {
                gemv_ring_rows1<T, G, 3, SetRef>(g, L, U, R, gw, nw, out, [&](uint32_t k) { trace_detail(a, r, k); });
                trace_detail(a, r, 23);
                return;
            }
        }
        gemv_ring<T, G, 3>(SD, g, L, U, R, gw, nw, out);
        trace_detail(a, r, 11);
        trace_clock(a, r, 15);
    });
    if (!ok && threadIdx.x == 0) raise_abort(a.abort_flag);
    return ok;
}

__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// ---------------------------------------------------------------------------
// Head: output_norm (batch-1 order, model.rs:1136-1143) + Q8 + head GEMV,
// logits and a (max, first index) pair per workgroup; workgroup 0 reduces
// the pairs to the greedy id.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool stage_head(const Cfg &a, Run r, const Lds &Lc, const uint64_t *xin, uint32_t *id_out,
                           uint32_t gw, uint32_t nw) {
    Lds L = Lc;
    set_act_k(L, a.ne);
    bool ok = true;
    const SetRef SH{&a.args->head};
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    with_kq(a.t_head, [&](auto T_, auto) {
        constexpr uint32_t T = decltype(T_)::value;
        Unit<T, 1> U[2];
        TileRef R[2];
        const Geo g = geo_of(SH);
        prefetch_ring<T, 1, 2>(SH, g, gw, nw, U, R);
        float4 wr[4];
        load_norm_w(a.out_norm, a.ne, wr);
        lds_barrier();
        if (xin) ok = poll_x(L, xin, a.ne, r.epoch, a.abort_flag);
        if (wg_any(!ok, L.vote)) { ok = false; return; }
        norm_q8(L, a.ne, a.eps, wr, true);
        auto out = [&](uint32_t, uint32_t row, float v) {
            gst(a.logits)[row] = v;
            amax_merge(best_v, best_i, v, row);
        };
        gemv_ring<T, 1, 2>(SH, g, L, U, R, gw, nw, out);
    });
    if (!ok) {
        if (threadIdx.x == 0) raise_abort(a.abort_flag);
        return false;
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    wave_argmax(best_v, best_i);
    float *sv = L.red + 400;
    uint32_t *si = reinterpret_cast<uint32_t *>(L.red + 408);
    if (lane == 0) {
        sv[wave] = best_v;
        si[wave] = best_i;
    }
    lds_barrier();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < MW; w++) amax_merge(best_v, best_i, sv[w], si[w]);
        ll_put(a.part + 2 * blockIdx.x, __float_as_uint(best_v), r.epoch);
        ll_put(a.part + 2 * blockIdx.x + 1, best_i, r.epoch);
    }
    if (blockIdx.x != 0) return true;
    // workgroup 0: reduce every workgroup's pair
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    ok = true;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += MT) {
        uint64_t wv = ll_get(a.part + 2 * b), wi = ll_get(a.part + 2 * b + 1);
        if (ok) ok = ll_wait(a.part + 2 * b, r.epoch, wv, a.abort_flag);
        if (ok) ok = ll_wait(a.part + 2 * b + 1, r.epoch, wi, a.abort_flag);
        amax_merge(bv, bi, __uint_as_float((uint32_t)wv), (uint32_t)wi);
    }
    PI_POLL_OR_LEAVE(ok);
    wave_argmax(bv, bi);
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    lds_barrier();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < MW; w++) amax_merge(bv, bi, sv[w], si[w]);
        if (bi == 0xFFFFFFFFu) bi = 0;
        *gst(a.tok_state) = bi;
        if (id_out) *gst(id_out) = bi;
    }
    return true;
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(MT, 1) void k_mega(const pi_mega_args *__restrict__ ap, const uint32_t *tok_src,
                                                uint32_t *id_out, uint32_t tok_imm, int32_t pos, uint32_t epoch,
                                                uint32_t flags) {
    extern __shared__ __align__(16) unsigned char smem[];
    const Cfg a = load_cfg(ap);
    Run r{pos, epoch, (flags & 1u) != 0, false};
    const bool head = (flags & 2u) != 0;
    const Lds L = carve(smem, a.ne, a.n_ff, a.n_ctx);
    // wave index in an SGPR: tile indices, tile bases and MatSet fields stay scalar
    const uint32_t gw = blockIdx.x * MW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = gridDim.x * MW;
    trace_mark(a, 0);
    // embedding of this launch's token (model.rs:857-869) into xt
    {
        const uint32_t tok = tok_src ? *gld(tok_src) : tok_imm;
        const uint8_t *row = a.embd + (uint64_t)tok * a.erow_bytes;
        unsigned char *rb = reinterpret_cast<unsigned char *>(L.hb);
        if ((a.erow_bytes & 3u) == 0) {
            for (uint32_t i = threadIdx.x; i < a.erow_bytes / 4; i += MT)
                reinterpret_cast<uint32_t *>(rb)[i] = gld(reinterpret_cast<const uint32_t *>(row))[i];
        } else {
            for (uint32_t i = threadIdx.x; i < a.erow_bytes; i += MT) rb[i] = gld(row)[i];
        }
        lds_barrier();
        for (uint32_t e = threadIdx.x; e < a.ne; e += MT) xt_set(L, e, embed_elem(rb, a.etype, e));
        lds_barrier();
    }
    trace_mark(a, 1);
    const uint32_t nb = gridDim.x;
    for (uint32_t l = 0; l < a.n_layer; l++) {
        const pi_mega_layer *Y = a.layers + l;
        r.detail = l == a.n_layer / 2;
        const uint64_t *xin = l == 0 ? nullptr : cload(&a.layers[l - 1].xo);
        if (!stage_qkv(a, r, Y, L, xin, gw, nw)) return;
        trace_mark(a, 2 + 5 * l);
        bool busy = false;   // attention or an attn_output tile in this layer
        {
            // long contexts split each head's positions into nseg segments, one
            // workgroup each (at most one item per workgroup: segments wait for
            // each other)
            const uint32_t n = (uint32_t)r.pos + 1;
            uint32_t nseg = (n + PI_MEGA_SEG_LEN - 1) / PI_MEGA_SEG_LEN;
            nseg = min(nseg, min(PI_MEGA_MAX_SEG, nb / a.n_head));
            nseg = max(nseg, 1u);
            const uint32_t nwg = max(nseg, 2u);   // at least the two chain workgroups
            busy = nb - 1 - blockIdx.x < a.n_head * nwg;
            for (uint32_t j = nb - 1 - blockIdx.x; j < a.n_head * nwg; j += nb)
                if (!stage_attn(a, r, Y, L, j % a.n_head, j / a.n_head, nseg, l)) return;
        }
        const bool attn = busy;
        busy = busy || blockIdx.x * MW < ms_total(SetRef{&Y->o});
        trace_mark(a, 3 + 5 * l);
        HUnits HU;
        h_units_fresh(HU);
        bool hpre = false;
        if (!stage_o(a, r, Y, L, gw, nw, HU, hpre, !attn)) return;
        trace_mark(a, 4 + 5 * l);
        if (!stage_ffn_up(a, r, Y, L, gw, nw, HU, hpre, !busy)) return;
        trace_mark(a, 5 + 5 * l);
        if (!stage_down(a, r, Y, L, gw, nw)) return;
        trace_mark(a, 6 + 5 * l);
    }
    r.detail = false;
    if (head) {
        if (!stage_head(a, r, L, cload(&a.layers[a.n_layer - 1].xo), id_out, gw, nw)) return;
        trace_mark(a, 2 + 5 * a.n_layer);
    }
}

}  // namespace

size_t pi_mega_lds_bytes(uint32_t ne, uint32_t n_ff, uint32_t n_ctx) { return lds_plan(ne, n_ff, n_ctx).total; }

bool pi_mega_h_blocks(uint32_t type, uint32_t upr, uint32_t ne, uint32_t n_ff, uint32_t n_ctx) {
    if (type != PI_TYPE_Q4_K || upr == 0 || upr > 64 || n_ff % 32) return false;
    const uint32_t rpw = 64 / upr;
    if (kHU * rpw < kHRowDots) return false;
    const LdsPlan p = lds_plan(ne, n_ff, n_ctx);
    return (uint64_t)MW * h_strip_floats(upr, QT<PI_TYPE_Q4_K>::TPB) * 4u <= p.strips - p.hb;
}

uint32_t pi_mega_blocks(int device, uint32_t ne, uint32_t n_ff, uint32_t n_ctx) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess) return 0;
    const size_t lds = pi_mega_lds_bytes(ne, n_ff, n_ctx);
    int occ = 0;
    auto kern = k_mega;
    if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, MT, lds) != hipSuccess || occ < 1) return 0;
    return (uint32_t)p.multiProcessorCount;
}

hipError_t pi_launch_mega(const pi_mega_args &a, const pi_mega_args *a_dev, const pi_mega_launch &l, bool neon,
                          bool head, uint32_t blocks, size_t lds, hipStream_t s) {
    if (!a_dev || l.epoch == 0 || l.epoch >= (1u << 26) || a.n_layer == 0 || a.n_layer > 63 || blocks == 0 || a.ne % 32 || a.ne / 32 > MT || a.n_ff / 32 > MT ||
        a.n_ff % 32 || a.half > 32 || a.n_head == 0 || a.n_kv == 0 || a.n_head % a.n_kv || l.pos < 0 ||
        (uint32_t)l.pos >= a.n_ctx || lds < pi_mega_lds_bytes(a.ne, a.n_ff, a.n_ctx))
        return hipErrorInvalidValue;
    const void *kern = (const void *)k_mega;
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const pi_mega_args *ap = a_dev;
    const uint32_t *tok_src = l.tok_src;
    uint32_t *id_out = l.id_out;
    uint32_t tok_imm = l.tok_imm;
    int32_t pos = l.pos;
    uint32_t epoch = l.epoch;
    uint32_t flags = (neon ? 1u : 0u) | (head ? 2u : 0u);
    void *args[] = {&ap, &tok_src, &id_out, &tok_imm, &pos, &epoch, &flags};
    return hipLaunchCooperativeKernel(kern, dim3(blocks), dim3(MT), args, (unsigned)lds, s);
}
