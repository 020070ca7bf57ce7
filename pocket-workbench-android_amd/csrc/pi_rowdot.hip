// Single-token f32 dot of the GGUF types without an int8 path (quant.rs:
// 377-441, dot_row_scalar's generic form): y[r] = 0 + w_0 x_0 + w_1 x_1 + ...
// over the row in element order, each product rounded before it is added,
// with w_j the f32 value dequant_row gives element j (quant.rs:102-359).
// The weights stay in their GGUF row layout.
//
// The add chain of a row is sequential; everything else is not.  A workgroup
// serves kRows rows: wavefront 0 keeps one add chain per row (lane = row),
// wavefronts 1-3 form the products.  Per step of 256 elements, producer lane
// (row, segment) dequantizes 32 consecutive elements of its row with the
// reference's float expressions, multiplies them by x and writes them to an
// LDS product buffer; after a barrier the chain lanes add the step's products
// in element order while the producers fill the other buffer.  A producer
// keeps the weights of its next kDepth steps in flight in registers.  The
// chains (one dependent add per element) set the pace once the producers keep
// up, so kRows is chosen for three producer wavefronts to match it.
//
// Q2_K, Q3_K and Q5_K follow the GGUF format's layout (qs advancing 32 bytes
// per 128 elements, hmask and qh indexed by the element's position within 32),
// where the reference's decoders index past their slices and panic
// (quant.rs:211, 254, 295-314).
#include <hip/hip_runtime.h>

#include "pi_common.h"
#include "pi_rowdot.h"

namespace {

// f16 -> f32 (v_cvt_f32_f16: exact, subnormals included, as util.rs:76-100)
__device__ __forceinline__ float h2f_bits(uint32_t bits) {
    const unsigned short b = (unsigned short)(bits & 0xFFFFu);
    _Float16 h;
    __builtin_memcpy(&h, &b, sizeof h);
    return (float)h;
}

// A whole 32-element block in registers: 32-bit words (4-aligned blocks), or
// words assembled from 16-bit loads (Q5_0's 22-byte blocks are 2-aligned).
template <uint32_t BB>
struct Blk {
    static constexpr uint32_t NW = (BB + 3) / 4;
    uint32_t w[NW];
    __device__ __forceinline__ void load(const uint8_t *p) {
        if constexpr (BB % 4 == 0) {
            const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
#pragma unroll
            for (uint32_t i = 0; i < NW; i++) w[i] = __builtin_nontemporal_load(q + i);
        } else {
            const uint16_t *q = reinterpret_cast<const uint16_t *>(p);
#pragma unroll
            for (uint32_t i = 0; i < NW; i++) {
                const uint32_t lo = __builtin_nontemporal_load(q + 2 * i);
                const uint32_t hi = (2 * i + 1) * 2 < BB ? (uint32_t)__builtin_nontemporal_load(q + 2 * i + 1) : 0u;
                w[i] = lo | (hi << 16);
            }
        }
    }
    __device__ __forceinline__ uint32_t byte(uint32_t i) const { return (w[i >> 2] >> (8 * (i & 3))) & 0xFFu; }
    __device__ __forceinline__ uint32_t u16(uint32_t i) const { return byte(i) | (byte(i + 1) << 8); }
    __device__ __forceinline__ uint32_t u32(uint32_t i) const { return u16(i) | (u16(i + 2) << 16); }
};

template <uint32_t T> struct TypeInfo;
template <> struct TypeInfo<PI_TYPE_Q4_1> { static constexpr uint32_t BE = 32, BB = 20; };
template <> struct TypeInfo<PI_TYPE_Q5_0> { static constexpr uint32_t BE = 32, BB = 22; };
template <> struct TypeInfo<PI_TYPE_Q5_1> { static constexpr uint32_t BE = 32, BB = 24; };
template <> struct TypeInfo<PI_TYPE_Q8_1> { static constexpr uint32_t BE = 32, BB = 36; };
template <> struct TypeInfo<PI_TYPE_Q2_K> { static constexpr uint32_t BE = 256, BB = 84; };
template <> struct TypeInfo<PI_TYPE_Q3_K> { static constexpr uint32_t BE = 256, BB = 110; };
template <> struct TypeInfo<PI_TYPE_Q5_K> { static constexpr uint32_t BE = 256, BB = 176; };
template <> struct TypeInfo<PI_TYPE_Q8_K> { static constexpr uint32_t BE = 256, BB = 292; };
template <> struct TypeInfo<PI_TYPE_BF16> { static constexpr uint32_t BE = 32, BB = 64; };   // 32 elements per step

// Bytes at a lane-dependent offset (the segment's part of a block).
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ uint32_t ld16(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}
// 16 bytes at a 4-byte aligned address, as one request.
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ void ld128(const uint8_t *p, uint32_t *d) {
    const u32x4a4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4a4 *>(p));
    d[0] = v.x;
    d[1] = v.y;
    d[2] = v.z;
    d[3] = v.w;
}
__device__ __forceinline__ uint32_t byte_of(const uint32_t *w, uint32_t i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xFFu; }
// Byte n (runtime, < 12) of three words, without indexing registers at run time.
__device__ __forceinline__ uint32_t byte12(const uint32_t (&w)[3], uint32_t n) {
    const uint32_t v = n < 4 ? w[0] : (n < 8 ? w[1] : w[2]);
    return (v >> (8 * (n & 3u))) & 0xFFu;
}

// What a producer lane holds of one step: the 32 elements of segment seg of
// its row's block (256-element types), or its own 32-element block.
// weights(seg, w) forms the 32 values dequant_row gives them.
template <uint32_t T> struct Seg;

template <uint32_t T> struct Seg32 {   // 32-element blocks: the whole block
    Blk<TypeInfo<T>::BB> B;
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t) { B.load(blk); }
};
template <> struct Seg<PI_TYPE_Q4_1> : Seg32<PI_TYPE_Q4_1> {};
template <> struct Seg<PI_TYPE_Q5_0> : Seg32<PI_TYPE_Q5_0> {};
template <> struct Seg<PI_TYPE_Q5_1> : Seg32<PI_TYPE_Q5_1> {};
template <> struct Seg<PI_TYPE_Q8_1> : Seg32<PI_TYPE_Q8_1> {};
template <> struct Seg<PI_TYPE_BF16> : Seg32<PI_TYPE_BF16> {};

template <> struct Seg<PI_TYPE_Q8_K> {   // f32 d, then 256 int8 quants (quant.rs:350-357)
    uint32_t d, q[8];
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t seg) {
        d = ld32(blk);
        ld128(blk + 4 + 32 * seg, q);
        ld128(blk + 20 + 32 * seg, q + 4);
    }
};
template <> struct Seg<PI_TYPE_Q2_K> {   // scales at 2 * seg, qs at 16 + 32 * (seg / 4), d and dmin at 80
    uint32_t dd, sc, qs[8];
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t seg) {
        dd = ld32(blk + 80);
        sc = ld16(blk + 2 * seg);
        ld128(blk + 16 + 32 * (seg >> 2), qs);
        ld128(blk + 32 + 32 * (seg >> 2), qs + 4);
    }
};
template <> struct Seg<PI_TYPE_Q3_K> {   // 110-byte blocks: 16-bit loads
    uint32_t hm[8], qs[8], sc[3], d;
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t seg) {
        auto two = [&](uint32_t off) { return ld16(blk + off) | (ld16(blk + off + 2) << 16); };
#pragma unroll
        for (int i = 0; i < 8; i++) hm[i] = two(4 * i);
#pragma unroll
        for (int i = 0; i < 8; i++) qs[i] = two(32 + 32 * (seg >> 2) + 4 * i);
#pragma unroll
        for (int i = 0; i < 3; i++) sc[i] = two(96 + 4 * i);
        d = ld16(blk + 108);
    }
};
template <> struct Seg<PI_TYPE_Q5_K> {   // d, dmin; 12 scale bytes; qh[32]; ql of pair seg / 2
    uint32_t dd, sc[3], qh[8], ql[8];
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t seg) {
        uint32_t h[4];
        ld128(blk, h);
        dd = h[0];
        sc[0] = h[1];
        sc[1] = h[2];
        sc[2] = h[3];
        ld128(blk + 16, qh);
        ld128(blk + 32, qh + 4);
        ld128(blk + 48 + 32 * (seg >> 1), ql);
        ld128(blk + 64 + 32 * (seg >> 1), ql + 4);
    }
};

// Byte b of v as a float (one v_cvt_f32_ubyte{b}).
__device__ __forceinline__ float ubyte_f(uint32_t v, uint32_t b) { return (float)((v >> (8 * b)) & 0xFFu); }
// Bits 0..3 of x moved to bit 0 of bytes 0..3.
__device__ __forceinline__ uint32_t spread4(uint32_t x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }
// The quant bytes are assembled a word (4 elements) at a time; each element's
// float is then formed with the reference's expression on an exact integer.
template <uint32_t T>
__device__ __forceinline__ void seg_weights(const Seg<T> &S, uint32_t seg, float (&w)[32]) {
    if constexpr (T == PI_TYPE_Q4_1 || T == PI_TYPE_Q5_0 || T == PI_TYPE_Q5_1) {
        // quant.rs:138-175: element j (< 16) is the low nibble of qs[j], j + 16 its high nibble; Q5 adds bit j of qh as 16
        const Blk<TypeInfo<T>::BB> &B = S.B;
        const float d = h2f_bits(B.u16(0));
        const float m = T == PI_TYPE_Q5_0 ? 0.0f : h2f_bits(B.u16(2));
        const uint32_t qh = T == PI_TYPE_Q5_0 ? B.u32(2) : (T == PI_TYPE_Q5_1 ? B.u32(4) : 0u);
        constexpr uint32_t qs0 = T == PI_TYPE_Q4_1 ? 4 : (T == PI_TYPE_Q5_0 ? 6 : 8);
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t v = B.u32(qs0 + 4 * i);   // qs bytes 4i .. 4i + 3
            uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;
            if constexpr (T != PI_TYPE_Q4_1) {
                lo |= spread4(qh >> (4 * i)) << 4;
                hi |= spread4(qh >> (16 + 4 * i)) << 4;
            }
#pragma unroll
            for (uint32_t b = 0; b < 4; b++) {
                if constexpr (T == PI_TYPE_Q5_0) {
                    w[4 * i + b] = (ubyte_f(lo, b) - 16.0f) * d;
                    w[16 + 4 * i + b] = (ubyte_f(hi, b) - 16.0f) * d;
                } else {
                    w[4 * i + b] = ubyte_f(lo, b) * d + m;
                    w[16 + 4 * i + b] = ubyte_f(hi, b) * d + m;
                }
            }
        }
    } else if constexpr (T == PI_TYPE_Q8_1) {
        // quant.rs:176-184: int8 quants at byte 4 times d
        const float d = h2f_bits(S.B.u16(0));
#pragma unroll
        for (uint32_t j = 0; j < 32; j++) w[j] = (float)(int8_t)S.B.byte(4 + j) * d;
    } else if constexpr (T == PI_TYPE_BF16) {   // quant.rs:122-126
#pragma unroll
        for (uint32_t j = 0; j < 32; j++) w[j] = __uint_as_float(S.B.u16(2 * j) << 16);
    } else if constexpr (T == PI_TYPE_Q8_K) {
        const float d = __uint_as_float(S.d);
#pragma unroll
        for (uint32_t j = 0; j < 32; j++) w[j] = (float)(int8_t)byte_of(S.q, j) * d;
    } else if constexpr (T == PI_TYPE_Q2_K) {
        // quant.rs:185-217's expressions: elements 32 * seg + 16 * half + l take
        // scale byte 2 * seg + half and bits 2 * (seg % 4) of qs byte 16 * half + l
        const float d = h2f_bits(S.dd), dmin = h2f_bits(S.dd >> 16);
        const uint32_t sh = 2 * (seg & 3u);
#pragma unroll
        for (uint32_t half = 0; half < 2; half++) {
            const uint32_t sc = (S.sc >> (8 * half)) & 0xFFu;
            const float dl = d * (float)(sc & 0xFu), ml = dmin * (float)(sc >> 4);
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t q = (S.qs[4 * half + i] >> sh) & 0x03030303u;
#pragma unroll
                for (uint32_t b = 0; b < 4; b++) w[16 * half + 4 * i + b] = dl * ubyte_f(q, b) - ml;
            }
        }
    } else if constexpr (T == PI_TYPE_Q3_K) {
        // quant.rs:218-259's expressions: scale g = 2 * seg + half; q = (qs bits
        // 2 * (seg % 4)) - 4 unless hmask bit seg of the element's byte is set
        const float d_all = h2f_bits(S.d);
        const uint32_t sh = 2 * (seg & 3u);
#pragma unroll
        for (uint32_t half = 0; half < 2; half++) {
            const uint32_t g = 2 * seg + half;
            const uint32_t lo4 = g < 8 ? (byte12(S.sc, g) & 0xFu) : (byte12(S.sc, g - 8) >> 4);
            const uint32_t hi2 = (byte12(S.sc, 8 + g % 4) >> (2 * (g / 4))) & 3u;
            const float dl = d_all * ((float)(int8_t)(lo4 | (hi2 << 4)) - 32.0f);
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                // 4 + q, 0..7: the two qs bits, and 4 when the hmask bit is set
                const uint32_t v = ((S.qs[4 * half + i] >> sh) & 0x03030303u) |
                                   (((S.hm[4 * half + i] >> seg) & 0x01010101u) << 2);
#pragma unroll
                for (uint32_t b = 0; b < 4; b++) w[16 * half + 4 * i + b] = dl * (ubyte_f(v, b) - 4.0f);
            }
        }
    } else {   // Q5_K, quant.rs:285-319's expressions: segment 2 p + hi
        const float d = h2f_bits(S.dd), dmin = h2f_bits(S.dd >> 16);
        const uint32_t j = seg;   // get_scale_min_k4 (quant.rs:80-86) on the 12 scale bytes
        uint32_t sv, mv;
        if (j < 4) {
            sv = byte12(S.sc, j) & 63u;
            mv = byte12(S.sc, j + 4) & 63u;
        } else {
            sv = (byte12(S.sc, j + 4) & 0xFu) | ((byte12(S.sc, j - 4) >> 6) << 4);
            mv = (byte12(S.sc, j + 4) >> 4) | ((byte12(S.sc, j) >> 6) << 4);
        }
        const float d1 = d * (float)sv, m1 = dmin * (float)mv;
        const uint32_t nsh = 4 * (seg & 1u), hb = seg;   // ql nibble; qh bit 2 p + hi = seg
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t q = ((S.ql[i] >> nsh) & 0x0F0F0F0Fu) | (((S.qh[i] >> hb) & 0x01010101u) << 4);
#pragma unroll
            for (uint32_t b = 0; b < 4; b++) w[4 * i + b] = d1 * ubyte_f(q, b) - m1;
        }
    }
}

constexpr uint32_t kRows = 24;                     // rows per workgroup (add chains in wavefront 0)
constexpr uint32_t kStep = 256;                    // elements per step
constexpr uint32_t kSeg = 32;                      // elements per producer task
constexpr uint32_t kSegs = kStep / kSeg;
constexpr uint32_t kPitch = kStep + 4;             // floats per row of a product buffer
constexpr uint32_t kThreads = 64 + kRows * kSegs;  // one chain wavefront, three producer wavefronts
constexpr int kDepth = 3;                          // steps of weights in flight per producer
static_assert(kThreads == 256, "four wavefronts");
constexpr uint32_t kProdFloats = 2 * kRows * kPitch;

// Workgroup barrier ordering LDS only: the producers' weight requests for the
// next steps stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Product buffer column of element e (< 256) of a step: the 4-element groups
// of a segment are rotated by the segment number, so the producers' 16-byte
// writes (eight segments of one row per eight lanes) fall on distinct banks.
__device__ __forceinline__ uint32_t prod_col(uint32_t seg, uint32_t g) { return seg * kSeg + 4 * ((g + seg) & 7u); }

template <uint32_t T>
__global__ __launch_bounds__(kThreads, 1) void k_gemv_row(const uint8_t *__restrict__ W, uint64_t row_bytes, uint32_t rows,
                                                          uint32_t k, const float *__restrict__ x, float *__restrict__ y) {
    constexpr uint32_t BE = TypeInfo<T>::BE, BB = TypeInfo<T>::BB;
    extern __shared__ __align__(16) float lds[];
    float *prod = lds, *xs = lds + kProdFloats;
    const uint32_t tid = threadIdx.x, r0 = blockIdx.x * kRows;
    // steps, and the step count rounded up to whole rounds of the producers'
    // ring (the padding steps only refill the ring and wait at the barrier)
    const uint32_t nsteps = (k + kStep - 1) / kStep, nb = k / BE;
    const uint32_t npad = (nsteps + kDepth - 1) / kDepth * kDepth;
    // x into LDS: all of a thread's loads are issued before its stores (one
    // memory round trip per 8 elements per thread, not one per element)
    if ((reinterpret_cast<uintptr_t>(x) & 15u) == 0) {
        const uint32_t k4 = k / 4;   // k % 32 == 0
        for (uint32_t base = 0; base < k4; base += kThreads * 8) {
            float4 v[8];
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) {
                const uint32_t q = min(base + tid + i * kThreads, k4 - 1);
                v[i] = reinterpret_cast<const float4 *>(x)[q];
            }
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) {
                const uint32_t q = base + tid + i * kThreads;
                if (q < k4) reinterpret_cast<float4 *>(xs)[q] = v[i];
            }
        }
    } else {
        for (uint32_t base = 0; base < k; base += kThreads * 8) {
            float v[8];
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) v[i] = x[min(base + tid + i * kThreads, k - 1)];
#pragma unroll
            for (uint32_t i = 0; i < 8; i++)
                if (base + tid + i * kThreads < k) xs[base + tid + i * kThreads] = v[i];
        }
    }
    if (tid < 64) {
        // ---- add chains: lane = row --------------------------------------
        const uint32_t lane = tid;
        float acc = 0.0f;
        lds_barrier();
        for (uint32_t s = 0; s <= npad; s++) {
            if (s >= 1 && s <= nsteps && lane < kRows) {
                const float *src = prod + ((s - 1) & 1u) * kRows * kPitch + lane * kPitch;
                const uint32_t nseg = min(kStep, k - (s - 1) * kStep) / kSeg;   // k % 32 == 0
                auto rd = [&](uint32_t sg, uint32_t g) { return *reinterpret_cast<const float4 *>(src + prod_col(sg, g)); };
                auto add8 = [&](const float4 (&v)[8]) {
#pragma unroll
                    for (uint32_t g = 0; g < 8; g++) {
                        acc = acc + v[g].x;
                        acc = acc + v[g].y;
                        acc = acc + v[g].z;
                        acc = acc + v[g].w;
                    }
                };
                if (nseg == kSegs) {   // a whole step: two segments of reads ahead of the adds
                    // (the scheduling barriers keep each batch of reads where it
                    // is written, ahead of the adds that do not need it)
                    float4 t[2][8];
#pragma unroll
                    for (uint32_t g = 0; g < 8; g++) t[0][g] = rd(0, g);
#pragma unroll
                    for (uint32_t g = 0; g < 8; g++) t[1][g] = rd(1, g);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (uint32_t sg = 0; sg < kSegs; sg++) {
                        add8(t[sg & 1]);
                        __builtin_amdgcn_sched_barrier(0);
                        if (sg + 2 < kSegs) {
#pragma unroll
                            for (uint32_t g = 0; g < 8; g++) t[sg & 1][g] = rd(sg + 2, g);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
                    for (uint32_t sg = 0; sg < nseg; sg++) {
                        float4 v[8];
#pragma unroll
                        for (uint32_t g = 0; g < 8; g++) v[g] = rd(sg, g);
                        add8(v);
                    }
                }
            }
            lds_barrier();
        }
        if (lane < kRows && r0 + lane < rows) y[r0 + lane] = acc;
        return;
    }
    // ---- producers: row r0 + rl, segment seg of each step -------------------
    const uint32_t t = tid - 64, rl = t / kSegs, seg = t % kSegs;
    const bool live = r0 + rl < rows;
    const uint8_t *row = W + (uint64_t)min(r0 + rl, rows - 1) * row_bytes;
    // block and segment of this lane at step s (clamped in bounds past the end)
    auto src = [&](uint32_t s) -> const uint8_t * {
        if constexpr (BE == kStep) return row + (uint64_t)min(s, nb - 1) * BB;
        else return row + (uint64_t)min(s * kSegs + seg, nb - 1) * BB;
    };
    // Every request is made at one place in the loop, in step order: round
    // -1 only requests the first kDepth steps, then each step refills its slot
    // after using it (past the end with a clamped block).  So the loads in
    // flight are always the next kDepth steps', oldest first, and a step waits
    // for its own only.
    Seg<T> ring[kDepth];
    lds_barrier();
    for (int s0 = -kDepth; s0 < (int)npad; s0 += kDepth) {
#pragma unroll
        for (int j = 0; j < kDepth; j++) {
            const int s = s0 + j;
            if (s >= 0) {
                const uint32_t e0 = (uint32_t)s * kStep + seg * kSeg;
                if (live && (uint32_t)s < nsteps && e0 < k) {
                    float w[32];
                    seg_weights<T>(ring[j], BE == kStep ? seg : 0u, w);
                    float *dst = prod + (s & 1) * kRows * kPitch + rl * kPitch;
#pragma unroll
                    for (uint32_t g = 0; g < 8; g++) {
                        const float4 x4 = *reinterpret_cast<const float4 *>(xs + e0 + 4 * g);
                        *reinterpret_cast<float4 *>(dst + prod_col(seg, g)) =
                            make_float4(w[4 * g] * x4.x, w[4 * g + 1] * x4.y, w[4 * g + 2] * x4.z, w[4 * g + 3] * x4.w);
                    }
                }
            }
            ring[j].load(src((uint32_t)(s + kDepth)), seg);
            if (s >= 0) lds_barrier();
        }
    }
    lds_barrier();   // the chains' last step
}

template <uint32_t T>
hipError_t launch_t(const uint8_t *w, uint64_t row_bytes, uint32_t rows, uint32_t k, const float *x, float *y, hipStream_t s) {
    if (k % 32 || k % TypeInfo<T>::BE || row_bytes != (uint64_t)(k / TypeInfo<T>::BE) * TypeInfo<T>::BB)
        return hipErrorInvalidValue;
    const size_t lds = pi_gemv_row_lds_bytes(k);
    hipError_t e = hipFuncSetAttribute((const void *)k_gemv_row<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_gemv_row<T>, dim3((rows + kRows - 1) / kRows), dim3(kThreads), lds, s, w, row_bytes, rows, k, x, y);
    return hipGetLastError();
}

}  // namespace

size_t pi_gemv_row_lds_bytes(uint32_t k) { return ((size_t)kProdFloats + k) * 4; }

hipError_t pi_launch_gemv_row(uint32_t type, const uint8_t *w, uint64_t row_bytes, uint32_t rows, uint32_t k,
                              const float *x, float *y, hipStream_t s) {
    if (!w || !x || !y || rows == 0 || k == 0) return hipErrorInvalidValue;
    switch (type) {
    case PI_TYPE_Q4_1: return launch_t<PI_TYPE_Q4_1>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_Q5_0: return launch_t<PI_TYPE_Q5_0>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_Q5_1: return launch_t<PI_TYPE_Q5_1>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_Q8_1: return launch_t<PI_TYPE_Q8_1>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_Q2_K: return launch_t<PI_TYPE_Q2_K>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_Q3_K: return launch_t<PI_TYPE_Q3_K>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_Q5_K: return launch_t<PI_TYPE_Q5_K>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_Q8_K: return launch_t<PI_TYPE_Q8_K>(w, row_bytes, rows, k, x, y, s);
    case PI_TYPE_BF16: return launch_t<PI_TYPE_BF16>(w, row_bytes, rows, k, x, y, s);
    default: return hipErrorInvalidValue;
    }
}
