// Single-token f32 dot of the GGUF types without an int8 path (quant.rs:
// 377-441, dot_row_scalar's generic form): y[r] = 0 + w_0 x_0 + w_1 x_1 + ...
// over the row in element order, each product rounded before it is added,
// with w_j the f32 value dequant_row gives element j (quant.rs:102-359).
// The weights stay in their GGUF row layout.  One lane per row: the lane reads
// its row block by block, forms each element with the reference's float
// expression and adds it to its own accumulator; x is staged in LDS and read
// by every lane at the same address.  The dependent add of each element sets
// the pace, so a launch is bound by its longest row, not by HBM.
//
// Q2_K, Q3_K and Q5_K follow the GGUF format's layout (qs advancing 32 bytes
// per 128 elements, hmask and qh indexed by the element's position within 32),
// where the reference's decoders index past their slices and panic
// (quant.rs:211, 254, 295-314).
#include <hip/hip_runtime.h>

#include "pi_common.h"
#include "pi_rowdot.h"

namespace {

constexpr uint32_t kRowThreads = 64;   // one wavefront per workgroup: rows spread over CUs

// f16 -> f32 (v_cvt_f32_f16: exact, subnormals included, as util.rs:76-100)
__device__ __forceinline__ float h2f_bits(uint32_t bits) {
    const unsigned short b = (unsigned short)(bits & 0xFFFFu);
    _Float16 h;
    __builtin_memcpy(&h, &b, sizeof h);
    return (float)h;
}

// Block bytes in registers: n 32-bit words (4-aligned blocks) or n/2 of them
// assembled from 16-bit loads (blocks of 22 and 110 bytes are 2-aligned).
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

// get_scale_min_k4 (quant.rs:80-86) of a K block whose 12 scale bytes start at byte 4.
template <uint32_t BB>
__device__ __forceinline__ void scale_min_k4(const Blk<BB> &B, uint32_t j, float &sc, float &m) {
    uint32_t s, mm;
    if (j < 4) {
        s = B.byte(4 + j) & 63u;
        mm = B.byte(4 + j + 4) & 63u;
    } else {
        s = (B.byte(4 + j + 4) & 0xFu) | ((B.byte(4 + j - 4) >> 6) << 4);
        mm = (B.byte(4 + j + 4) >> 4) | ((B.byte(4 + j) >> 6) << 4);
    }
    sc = (float)s;
    m = (float)mm;
}

// Adds the block's elements times x (LDS, this block's elements) to acc in
// element order.
template <uint32_t T>
__device__ __forceinline__ void block_dot(const Blk<TypeInfo<T>::BB> &B, const float *xb, float &acc) {
    auto add4 = [&](uint32_t j, float w0, float w1, float w2, float w3) {
        const float4 x4 = *reinterpret_cast<const float4 *>(xb + j);
        acc = acc + w0 * x4.x;
        acc = acc + w1 * x4.y;
        acc = acc + w2 * x4.z;
        acc = acc + w3 * x4.w;
    };
    if constexpr (T == PI_TYPE_Q4_1 || T == PI_TYPE_Q5_0 || T == PI_TYPE_Q5_1) {
        // quant.rs:138-175: element j (< 16) is the low nibble of qs[j], j + 16 its high nibble; Q5 adds bit j of qh as 16
        const float d = h2f_bits(B.u16(0));
        const float m = T == PI_TYPE_Q5_0 ? 0.0f : h2f_bits(B.u16(2));
        const uint32_t qh = T == PI_TYPE_Q5_0 ? B.u32(2) : (T == PI_TYPE_Q5_1 ? B.u32(4) : 0u);
        constexpr uint32_t qs0 = T == PI_TYPE_Q4_1 ? 4 : (T == PI_TYPE_Q5_0 ? 6 : 8);
        float w[32];
#pragma unroll
        for (uint32_t j = 0; j < 16; j++) {
            const uint32_t v = B.byte(qs0 + j);
            uint32_t lo = v & 0x0Fu, hi = v >> 4;
            if constexpr (T != PI_TYPE_Q4_1) {
                lo |= ((qh >> j) << 4) & 0x10u;
                hi |= (qh >> (j + 12)) & 0x10u;
            }
            if constexpr (T == PI_TYPE_Q5_0) {
                w[j] = ((float)lo - 16.0f) * d;
                w[j + 16] = ((float)hi - 16.0f) * d;
            } else {
                w[j] = (float)lo * d + m;
                w[j + 16] = (float)hi * d + m;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 32; j += 4) add4(j, w[j], w[j + 1], w[j + 2], w[j + 3]);
    } else if constexpr (T == PI_TYPE_Q8_1) {
        // quant.rs:176-184: int8 quants at byte 4 times d
        const float d = h2f_bits(B.u16(0));
#pragma unroll
        for (uint32_t j = 0; j < 32; j += 4) {
            float w[4];
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) w[i] = (float)(int8_t)B.byte(4 + j + i) * d;
            add4(j, w[0], w[1], w[2], w[3]);
        }
    } else if constexpr (T == PI_TYPE_Q8_K) {
        // quant.rs:350-357: f32 d, then 256 int8 quants
        const float d = __uint_as_float(B.u32(0));
#pragma unroll
        for (uint32_t j = 0; j < 256; j += 4) {
            float w[4];
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) w[i] = (float)(int8_t)B.byte(4 + j + i) * d;
            add4(j, w[0], w[1], w[2], w[3]);
        }
    } else if constexpr (T == PI_TYPE_Q2_K) {
        // quant.rs:185-217's expressions; qs (byte 16) advances 32 bytes per 128 elements
        const float d = h2f_bits(B.u16(80)), dmin = h2f_bits(B.u16(82));
#pragma unroll
        for (uint32_t hh = 0; hh < 2; hh++)
#pragma unroll
            for (uint32_t s = 0; s < 4; s++)
#pragma unroll
                for (uint32_t half = 0; half < 2; half++) {
                    const uint32_t sc = B.byte(8 * hh + 2 * s + half);
                    const float dl = d * (float)(sc & 0xFu), ml = dmin * (float)(sc >> 4);
                    const uint32_t e0 = 128 * hh + 32 * s + 16 * half;
#pragma unroll
                    for (uint32_t l = 0; l < 16; l += 4) {
                        float w[4];
#pragma unroll
                        for (uint32_t i = 0; i < 4; i++)
                            w[i] = dl * (float)((B.byte(16 + 32 * hh + 16 * half + l + i) >> (2 * s)) & 3u) - ml;
                        add4(e0 + l, w[0], w[1], w[2], w[3]);
                    }
                }
    } else if constexpr (T == PI_TYPE_Q3_K) {
        // quant.rs:218-259's expressions; hmask (byte 0) indexed by l, bit 4 * hh + s;
        // qs (byte 32) advances 32 bytes per 128 elements; 6-bit scales at byte 96
        const float d_all = h2f_bits(B.u16(108));
#pragma unroll
        for (uint32_t hh = 0; hh < 2; hh++)
#pragma unroll
            for (uint32_t s = 0; s < 4; s++)
#pragma unroll
                for (uint32_t half = 0; half < 2; half++) {
                    const uint32_t g = 8 * hh + 2 * s + half;
                    const uint32_t lo4 = g < 8 ? (B.byte(96 + g) & 0xFu) : (B.byte(96 + g - 8) >> 4);
                    const uint32_t hi2 = (B.byte(96 + 8 + g % 4) >> (2 * (g / 4))) & 3u;
                    const float dl = d_all * ((float)(int8_t)(lo4 | (hi2 << 4)) - 32.0f);
                    const uint32_t e0 = 128 * hh + 32 * s + 16 * half;
#pragma unroll
                    for (uint32_t l = 0; l < 16; l += 4) {
                        float w[4];
#pragma unroll
                        for (uint32_t i = 0; i < 4; i++) {
                            const uint32_t li = 16 * half + l + i;
                            const int hi = ((B.byte(li) >> (4 * hh + s)) & 1u) ? 0 : 4;
                            const int q = (int)((B.byte(32 + 32 * hh + li) >> (2 * s)) & 3u) - hi;
                            w[i] = dl * (float)q;
                        }
                        add4(e0 + l, w[0], w[1], w[2], w[3]);
                    }
                }
    } else if constexpr (T == PI_TYPE_Q5_K) {
        // quant.rs:285-319's expressions; qh (byte 16) indexed by l, bits 2p and 2p + 1;
        // ql (byte 48) advances 32 bytes per 64 elements
        const float d = h2f_bits(B.u16(0)), dmin = h2f_bits(B.u16(2));
#pragma unroll
        for (uint32_t p = 0; p < 4; p++)
#pragma unroll
            for (uint32_t hi = 0; hi < 2; hi++) {
                float sc, m;
                scale_min_k4(B, 2 * p + hi, sc, m);
                const float d1 = d * sc, m1 = dmin * m;
#pragma unroll
                for (uint32_t l = 0; l < 32; l += 4) {
                    float w[4];
#pragma unroll
                    for (uint32_t i = 0; i < 4; i++) {
                        const uint32_t nib = (B.byte(48 + 32 * p + l + i) >> (4 * hi)) & 0xFu;
                        const uint32_t q = nib + (((B.byte(16 + l + i) >> (2 * p + hi)) & 1u) ? 16u : 0u);
                        w[i] = d1 * (float)q - m1;
                    }
                    add4(64 * p + 32 * hi + l, w[0], w[1], w[2], w[3]);
                }
            }
    } else {   // BF16, 32 elements (quant.rs:122-126)
#pragma unroll
        for (uint32_t j = 0; j < 32; j += 4) {
            float w[4];
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) w[i] = __uint_as_float(B.u16(2 * (j + i)) << 16);
            add4(j, w[0], w[1], w[2], w[3]);
        }
    }
}

template <uint32_t T>
__global__ __launch_bounds__(kRowThreads) void k_gemv_row(const uint8_t *__restrict__ W, uint64_t row_bytes, uint32_t rows,
                                                          uint32_t k, const float *__restrict__ x, float *__restrict__ y) {
    constexpr uint32_t BE = TypeInfo<T>::BE, BB = TypeInfo<T>::BB;
    extern __shared__ __align__(16) float xs[];
    for (uint32_t i = threadIdx.x; i < k; i += kRowThreads) xs[i] = x[i];
    __syncthreads();
    const uint32_t r = blockIdx.x * kRowThreads + threadIdx.x;
    if (r >= rows) return;
    const uint8_t *row = W + (uint64_t)r * row_bytes;
    const uint32_t nb = k / BE;
    float acc = 0.0f;
    Blk<BB> cur, nxt;
    cur.load(row);
    for (uint32_t b = 0; b < nb; b++) {
        if (b + 1 < nb) nxt.load(row + (uint64_t)(b + 1) * BB);   // the next block is requested before this one is used
        block_dot<T>(cur, xs + b * BE, acc);
        cur = nxt;
    }
    y[r] = acc;
}

template <uint32_t T>
hipError_t launch_t(const uint8_t *w, uint64_t row_bytes, uint32_t rows, uint32_t k, const float *x, float *y, hipStream_t s) {
    if (k % TypeInfo<T>::BE || row_bytes != (uint64_t)(k / TypeInfo<T>::BE) * TypeInfo<T>::BB) return hipErrorInvalidValue;
    const size_t lds = (size_t)k * 4;
    hipError_t e = hipFuncSetAttribute((const void *)k_gemv_row<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_gemv_row<T>, dim3((rows + kRowThreads - 1) / kRowThreads), dim3(kRowThreads), lds, s, w, row_bytes,
                       rows, k, x, y);
    return hipGetLastError();
}

}  // namespace

size_t pi_gemv_row_lds_bytes(uint32_t k) { return (size_t)k * 4; }

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
