// Batched projection GEMM of the engine step, gfx950:
//   y[b][o] = sum_i W[o][i] * x[b][i]
// the product QuantKernels.MatMulBatch(type, W, x, y, inDim, outDim, batch)
// computes around the attention step (PagedTransformerRunner.cs:601-603,659).
// W holds out_dim rows of in_dim weights (the GGUF [in, out] layout) as F32,
// Q8_0 (blocks of 32 int8 with an fp16 scale d: w = d * q), or the K-quant
// super-blocks Q4_K and Q6_K (256 weights each, decoded further down).
//
// Two forms.  The fp32 form (matmul_batch_kernel, every F32 product and the
// quantized ones too small for the fp16 forms): every weight is exact in fp32
// (Q8_0's d * q has at most 19 significant bits), and the products run on
// v_mfma_f32_16x16x4f32 with fp32 accumulation, so no operand is rounded below
// fp32.  The fp16 forms
// (matmul_f16_kernel and the small-batch variants for at most 64 batch rows,
// described further down) run Q8_0, Q4_K and Q6_K blocks on fp16 matrix steps
// with the quants exact in fp16 and x as a scaled fp16 pair.
//
// fp32 form:
// A workgroup (four waves) owns 64 weight rows (16 per wave, MFMA M) and 64
// batch rows (four 16-column MFMA tiles, N) over a range of K, in 64-wide
// chunks.  Each chunk of x is staged once in LDS and serves all four waves;
// lane group g = lane / 16 supplies k = k0 + 16 g + s at step s of the chunk
// in both operands, so each lane reads 16 contiguous weights of its row from
// memory and 16 contiguous inputs of a batch row from LDS.  The next chunk's
// weights and x load while the current chunk computes.  When the host splits
// K over grid.z workgroups, each writes its sums to a partial buffer and a
// second kernel adds the partials in order, so results do not depend on
// timing.
#include <cfloat>
#include <type_traits>

#include "gsp_epilogue.h"
#include "gsp_internal.h"

namespace gsp {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kMmThreads = 256;
constexpr int kMmRowsWg = 64;  // weight rows per workgroup, 16 per wave

// The lane's 16 weights of row o at columns k0 + 16 g .. + 15, in two steps:
// load_raw issues the loads into registers, expand turns them into floats.
// A chunk's raw words are loaded one chunk ahead and expanded only when the
// chunk is computed, so the loads have a whole chunk of products to arrive.
template <int WT>
struct WRaw;

template <>
struct WRaw<kWeightF32> {
    f4 v[4];
};

// Q8_0: five dwords holding the lane's 16 bytes, and the dword holding its scale.
template <>
struct WRaw<kWeightQ8_0> {
    uint32_t dw[5];
    uint32_t sw;
};

__device__ __forceinline__ void load_raw(WRaw<kWeightF32>& r, const MatmulArgs& a, int o, int k0, int g) {
    const f4* p = reinterpret_cast<const f4*>(static_cast<const float*>(a.w) + (int64_t)o * a.in_dim + k0 + 16 * g);
#pragma unroll
    for (int j = 0; j < 4; ++j) r.v[j] = p[j];
}

__device__ __forceinline__ void expand(float (&w)[16], const WRaw<kWeightF32>& r, int) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * j + e] = r.v[j][e];
}

// Q8_0: a 64-wide chunk of a row is two 34-byte blocks, 68 bytes starting at a
// multiple of 4 (in_dim is a multiple of 64).  Lane group g's 16 values sit at
// bytes 2 + 16 g (g < 2, first block) or 36 + 16 (g - 2) (second block): the
// lane reads the five dwords from (byte 0, 16, 36, 52) and shifts out the
// first 2 (g < 2) or 0 bytes.  Its block's scale is the low half of dword 0
// or the high half of dword 8.  Every dword read lies inside the chunk.
__device__ __forceinline__ void load_raw(WRaw<kWeightQ8_0>& r, const MatmulArgs& a, int o, int k0, int g) {
    const int64_t row_bytes = (int64_t)(a.in_dim / 32) * 34;
    const uint32_t* cw = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(a.w) + (int64_t)o * row_bytes +
                                                           (int64_t)(k0 / 64) * 68);
    const int first = g < 2 ? 4 * g : 9 + 4 * (g - 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.dw[i] = cw[first + i];
    r.dw[4] = cw[g < 2 ? first + 4 : first + 3];  // only read as the high half of a 2-byte shift
    r.sw = cw[g < 2 ? 0 : 8];
}

__device__ __forceinline__ void expand(float (&w)[16], const WRaw<kWeightQ8_0>& r, int g) {
    const int shift = g < 2 ? 2 : 0;
    const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)(g < 2 ? (r.sw & 0xFFFFu) : (r.sw >> 16)));
    const float d = (float)dh;
    const float bias = -128.0f * d;  // w = d * (u - 128) for the byte u = q ^ 0x80, exact in one fma
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t qd = __builtin_amdgcn_alignbyte(r.dw[i + 1], r.dw[i], shift) ^ 0x80808080u;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * i + e] = fmaf((float)((qd >> (8 * e)) & 0xFFu), d, bias);
    }
}

// K-quants: super-blocks of 256 weights in the public GGML layouts.  A
// 64-wide chunk lies inside one super-block; lane group g's 16 weights are
// columns 16 g .. 16 g + 15 of the chunk.  Every weight is decoded to the
// float32 value the layout defines, in its own order of operations, so the
// products stay exact fp32 products as for F32 weights.
//
// Q4_K (144 bytes: fp16 d, fp16 dmin, 12 bytes of 6-bit scales and mins, 128
// bytes of 4-bit quants): chunk p of the super-block is sub-blocks 2 p (the low
// nibbles of quant bytes 32 p .. 32 p + 31) and 2 p + 1 (their high nibbles),
// weight = (d * sc) * q - dmin * m with one rounding.  The lane reads the
// header dword, the three scale dwords and the four dwords of its 16 quant
// bytes (32 p + 16 (g % 2)); super-blocks are 4-byte aligned.
template <>
struct WRaw<kWeightQ4_K> {
    uint32_t hdr;    // d | dmin << 16
    uint32_t sc[3];  // the 12 packed scale/min bytes
    uint32_t q[4];   // the lane's 16 quant bytes
    int j;           // the lane's sub-block, 0..7
};

__device__ __forceinline__ void load_raw(WRaw<kWeightQ4_K>& r, const MatmulArgs& a, int o, int k0, int g) {
    const int64_t row_bytes = (int64_t)(a.in_dim / 256) * 144;
    const uint32_t* bw = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(a.w) + (int64_t)o * row_bytes +
                                                           (int64_t)(k0 / 256) * 144);
    const int p = (k0 & 255) >> 6;
    r.hdr = bw[0];
#pragma unroll
    for (int i = 0; i < 3; ++i) r.sc[i] = bw[1 + i];
    const int qw = 4 + 8 * p + 4 * (g & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.q[i] = bw[qw + i];
    r.j = 2 * p + (g >> 1);
}

__device__ __forceinline__ uint32_t sc_byte(const uint32_t (&sc)[3], int k) {
    const uint32_t w = k < 4 ? sc[0] : k < 8 ? sc[1] : sc[2];
    return (w >> (8 * (k & 3))) & 0xFFu;
}

// The six-bit scale and min of sub-block j: bytes j and j + 4 for j < 4;
// else the nibbles of byte j + 4 with the top two bits of bytes j - 4
// (scale) and j (min).
__device__ __forceinline__ void q4k_scale_min(const uint32_t (&sc)[3], int j, uint32_t& scv, uint32_t& mv) {
    if (j < 4) {
        scv = sc_byte(sc, j) & 63u;
        mv = sc_byte(sc, j + 4) & 63u;
    } else {
        scv = (sc_byte(sc, j + 4) & 0xFu) | ((sc_byte(sc, j - 4) >> 6) << 4);
        mv = (sc_byte(sc, j + 4) >> 4) | ((sc_byte(sc, j) >> 6) << 4);
    }
}

__device__ __forceinline__ void expand(float (&w)[16], const WRaw<kWeightQ4_K>& r, int g) {
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.hdr & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.hdr >> 16));
    uint32_t scv, mv;
    q4k_scale_min(r.sc, r.j, scv, mv);
    const float d1 = d * (float)scv;   // exact
    const float m1 = dmin * (float)mv;  // exact
    const int shift = 4 * (g >> 1);     // low nibbles for sub-block 2 p, high for 2 p + 1
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) w[4 * i + e] = fmaf(d1, (float)((r.q[i] >> (8 * e + shift)) & 0xFu), -m1);
}

// Q6_K (210 bytes: 128 bytes of the quants' low 4 bits, 64 bytes of their
// high 2 bits, 16 int8 scales, fp16 d): chunk cc of the super-block is half
// n = cc / 2, and lane group g takes quarter c = 2 (cc % 2) + g / 2, weights
// l0 .. l0 + 15 of it (l0 = 16 (g % 2)): low bytes 64 n + 32 (c % 2) + l
// (low nibble for c < 2, high for c >= 2), bits 2 c .. 2 c + 1 of high bytes
// 32 n + l, scale 8 n + l / 16 + 2 c; weight = (d * scale) * (q - 32).
// Super-blocks are only 2-byte aligned (210 bytes), so the lane reads 16-bit
// words.
template <>
struct WRaw<kWeightQ6_K> {
    uint32_t lo[4];  // the 16 low-nibble bytes (pairs of 16-bit words)
    uint32_t hi[4];  // the 16 high-bit bytes
    uint32_t sd;     // the scale byte | d << 16
    int c;           // the lane's quarter, 0..3
};

__device__ __forceinline__ void load_raw(WRaw<kWeightQ6_K>& r, const MatmulArgs& a, int o, int k0, int g) {
    const int64_t row_bytes = (int64_t)(a.in_dim / 256) * 210;
    const uint8_t* blk = static_cast<const uint8_t*>(a.w) + (int64_t)o * row_bytes + (int64_t)(k0 / 256) * 210;
    const uint16_t* bh = reinterpret_cast<const uint16_t*>(blk);
    const int cc = (k0 & 255) >> 6;
    const int n = cc >> 1;
    const int c = 2 * (cc & 1) + (g >> 1);
    const int l0 = 16 * (g & 1);
    const int lo_h = (64 * n + 32 * (c & 1) + l0) >> 1;  // in 16-bit words
    const int hi_h = (128 + 32 * n + l0) >> 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r.lo[i] = (uint32_t)bh[lo_h + 2 * i] | ((uint32_t)bh[lo_h + 2 * i + 1] << 16);
        r.hi[i] = (uint32_t)bh[hi_h + 2 * i] | ((uint32_t)bh[hi_h + 2 * i + 1] << 16);
    }
    r.sd = (uint32_t)blk[192 + 8 * n + (l0 >> 4) + 2 * c] | ((uint32_t)bh[104] << 16);
    r.c = c;
}

__device__ __forceinline__ void expand(float (&w)[16], const WRaw<kWeightQ6_K>& r, int) {
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.sd >> 16));
    const float ds = d * (float)(int8_t)(r.sd & 0xFFu);  // exact
    const int nib = 4 * (r.c >> 1);
    const int hb = 2 * r.c;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int q = (int)(((r.lo[i] >> (8 * e + nib)) & 0xFu) | (((r.hi[i] >> (8 * e + hb)) & 3u) << 4)) - 32;
            w[4 * i + e] = ds * (float)q;
        }
}

template <int WT>
__global__ __launch_bounds__(kMmThreads, 2) void matmul_batch_kernel(MatmulArgs a) {
    // The chunk of x (64 batch rows x 64 k), two buffers; rows padded by one
    // 16-byte word so that the 16 lanes of one read hit distinct banks.
    __shared__ f4 xs[2][64][17];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int m = lane & 15;  // weight row of the wave's tile (A) and batch row within a tile (B)
    const int g = lane >> 4;  // K group
    const int o0 = blockIdx.x * kMmRowsWg + 16 * wave;
    const int b0 = blockIdx.y * 64;
    const int nt = min(4, (a.batch - b0 + 15) >> 4);  // batch tiles in use
    const int o = min(o0 + m, a.out_dim - 1);          // rows past out_dim load row out_dim - 1, never stored
    const int chunks = a.in_dim / 64;
    const int c_begin = blockIdx.z * a.chunks_per_split;
    const int c_end = min(chunks, c_begin + a.chunks_per_split);

    // x staging: thread tid moves batch row tid / 4, columns 16 (tid % 4) .. + 15.
    const int xr = tid >> 2;
    const int xq = tid & 3;
    const f4* xsrc = reinterpret_cast<const f4*>(a.x + (int64_t)min(b0 + xr, a.batch - 1) * a.in_dim + 16 * xq);
    f4 xreg[4];
    WRaw<WT> wraw;
    auto load_chunk = [&](int c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xreg[j] = xsrc[16 * c + j];
        load_raw(wraw, a, o, 64 * c, g);
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xs[buf][xr][4 * xq + j] = xreg[j];
    };

    f4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    if (c_begin < c_end) {
        load_chunk(c_begin);
        store_x(0);
    }
    __syncthreads();
    for (int c = c_begin; c < c_end; ++c) {
        const int buf = (c - c_begin) & 1;
        float w[16];
        expand(w, wraw, g);
        const bool more = c + 1 < c_end;
        if (more) load_chunk(c + 1);  // the next chunk loads while this one computes
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (t < nt) {
                float xv[16];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f4 v = xs[buf][16 * t + m][4 * g + j];
#pragma unroll
                    for (int e = 0; e < 4; ++e) xv[4 * j + e] = v[e];
                }
#pragma unroll
                for (int s2 = 0; s2 < 16; ++s2)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[s2], xv[s2], acc[t], 0, 0, 0);
            }
        }
        if (more) store_x(buf ^ 1);  // the other buffer's last readers passed the previous barrier
        __syncthreads();
    }

    // Lane holds weight rows o0 + 4 g + r of batch row b0 + 16 t + m.
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int b = b0 + 16 * t + m;
        if (t >= nt || b >= a.batch) continue;
        float* dst = a.split_out ? a.split_out + ((int64_t)blockIdx.z * a.batch + b) * a.out_dim
                                 : a.y + (int64_t)b * a.out_dim;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int oo = o0 + 4 * g + r;
            if (oo < a.out_dim) dst[oo] = acc[t][r];
        }
    }
}

// ---- Q8_0 weights on the fp16 matrix cores ----------------------------------
//
// One Q8_0 block (32 weights of a row) is one K step of v_mfma_f32_16x16x32_f16:
// its int8 values are exact in fp16, and x enters as a pair x = 2^e (x_hi +
// x_lo) of fp16 halves, scaled per batch row so that the row's largest |x|
// lies in [2^12, 2^13) (the pair then carries ~22 significant bits and x_lo
// stays a normal fp16 number).  A block's two products go into a fresh
// accumulator, which the block's scale d then adds into the running sum;
// 2^e multiplies the finished row.  The products are exact in fp32, so the
// result differs from the fp32 kernel's only by summation order and the
// ~2^-22 relative truncation of x.
//
// Tile layout (M = batch rows, N = weight rows): A lane l holds
// x[batch 16 t + l % 16][k0 + 8 (l / 16) .. + 7], B lane l holds
// q[row l % 16][the same k], and the result lane holds
// y[batch 16 t + 4 (l / 16) + r][row l % 16]: the lane's own weight row, so
// its block scale is its own.

// x of one batch row as scaled fp16 pairs: one workgroup per row, four
// elements per access (in_dim is a multiple of 64, rows 16-byte aligned).
// With kSums (Q4_K weights) it also writes each 32-wide block's sum of the
// scaled x, xsum[b * (in_dim / 32) + block], for the weights' min term.
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
template <bool kSums>
__global__ __launch_bounds__(kMmThreads) void matmul_split_x_kernel(MatmulArgs a) {
    __shared__ float red[kMmThreads / 64];
    const int b = blockIdx.x;
    const int n4 = a.in_dim / 4;
    const f4* xr = reinterpret_cast<const f4*>(a.x + (int64_t)b * a.in_dim);
    // Rows of up to 16384 values stay in registers between the two passes
    // (every load issued at once, indexes clamped); longer rows are read twice.
    constexpr int kHeld = 16;
    const bool held = n4 <= kHeld * kMmThreads;
    f4 hv[kHeld];
    float mx = 0.f;
    if (held) {
#pragma unroll
        for (int j = 0; j < kHeld; ++j)
            if (kMmThreads * j < n4) hv[j] = xr[min((int)threadIdx.x + kMmThreads * j, n4 - 1)];
#pragma unroll
        for (int j = 0; j < kHeld; ++j)
            if (kMmThreads * j < n4)
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(hv[j][0]), fabsf(hv[j][1])), fmaxf(fabsf(hv[j][2]), fabsf(hv[j][3]))));
    } else {
#pragma unroll 4
        for (int i = threadIdx.x; i < n4; i += kMmThreads) {
            const f4 v = xr[i];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // e with mx * 2^-e in [2^12, 2^13), clamped to [-126, 115] so that 2^-e
    // and 2^e stay normal floats.  The ceiling covers every finite row (ex is
    // at most 128), so no finite x overflows fp16; rows below 2^-113 keep
    // their absolute fp16 rounding only.
    int ex = 0;
    if (mx > 0.f && mx <= FLT_MAX) (void)frexpf(mx, &ex);
    const int e = mx > 0.f ? (mx <= FLT_MAX ? min(115, max(-126, ex - 13)) : 115) : 0;
    const float down = ldexpf(1.0f, -e);
    h4v* xh = reinterpret_cast<h4v*>(static_cast<_Float16*>(a.xh) + (int64_t)b * a.in_dim);
    h4v* xl = reinterpret_cast<h4v*>(static_cast<_Float16*>(a.xl) + (int64_t)b * a.in_dim);
    auto put = [&](int i, f4 raw) {
        const f4 v = raw * down;
        const h4v h = __builtin_convertvector(v, h4v);
        // An infinite element rides on its hi half alone (Inf - Inf would make
        // the lo half NaN), as it would through the fp32 form.
        f4 l = v - __builtin_convertvector(h, f4);
#pragma unroll
        for (int c = 0; c < 4; ++c) l[c] = __builtin_isinf(v[c]) ? 0.f : l[c];
        const h4v lh = __builtin_convertvector(l, h4v);
        xh[i] = h;
        xl[i] = lh;
        if constexpr (kSums) {
            // Eight consecutive threads hold a block's 32 values (n4 is a multiple
            // of 16, so a group is active or inactive as a whole): a tree over it.
            float sm = (v[0] + v[1]) + (v[2] + v[3]);
            sm += __shfl_xor(sm, 1);
            sm += __shfl_xor(sm, 2);
            sm += __shfl_xor(sm, 4);
            if ((i & 7) == 0) a.xsum[(int64_t)b * (a.in_dim / 32) + (i >> 3)] = sm;
        }
    };
    if (held) {
#pragma unroll
        for (int j = 0; j < kHeld; ++j) {
            const int i = threadIdx.x + kMmThreads * j;
            if (i < n4) put(i, hv[j]);
        }
    } else if constexpr (kSums) {
        // The block sums' lane exchanges keep this loop rolled.
        for (int i = threadIdx.x; i < n4; i += kMmThreads) put(i, xr[i]);
    } else {
#pragma unroll 4
        for (int i = threadIdx.x; i < n4; i += kMmThreads) put(i, xr[i]);
    }
    if (threadIdx.x == 0) a.xexp[b] = e;
}

// The small-batch form's pre-pass: workgroup (b, z) turns batch row b's K
// range z (the product kernel's range, chunks_per_split chunks of 64) into
// scaled fp16 pairs in the order the product kernel's A operands are read,
// tile by tile: for M tile t (batch rows 16 t ..) and chunk c, 4096 bytes as
// [block][hi, lo][lane g * 16 + m][8 halves], the halves
// x[16 t + m][64 c + 32 block + 8 g ..], so that a wave loads one operand of
// one block as 1 KB in one instruction.  Each range has an exponent of its
// own, xexp[z][b]
// (the product kernel scales each range's partial by it).  A range's largest
// |x| is at most its row's, so every element keeps at least the per-row
// form's precision.  One f4 per thread and a single load round trip: for
// Qwen2.5-7B's 3584-wide rows at 64 batch rows that is 448 workgroups of 128
// elements' worth each instead of 64 workgroups walking whole rows.
// With kSums (Q4_K weights) it also writes each 32-wide block's sum of the
// scaled x, xsum[(z * 2 chunks_per_split + block of the range) * 64 + b], for
// the weights' min term.
// kSlots f4 per thread: ranges of up to 16 kSlots chunks.
template <bool kSums, int kSlots>
__global__ __launch_bounds__(kMmThreads) void matmul_split_x_range_kernel(MatmulArgs a) {
    __shared__ float red[kMmThreads / 64];
    const int b = blockIdx.x;
    const int z = blockIdx.y;
    const int i0 = z * a.chunks_per_split * 16;  // first f4 of the range
    const int n4 = min(a.in_dim / 4, i0 + a.chunks_per_split * 16) - i0;  // host: at most kSlots * kMmThreads
    const int t = threadIdx.x;
    const f4* xr = reinterpret_cast<const f4*>(a.x + (int64_t)b * a.in_dim) + i0;
    f4 raw[kSlots];
    float mx = 0.f;
#pragma unroll
    for (int sl = 0; sl < kSlots; ++sl) {
        const int tt = t + sl * kMmThreads;
        raw[sl] = tt < n4 ? xr[tt] : f4{0.f, 0.f, 0.f, 0.f};
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(raw[sl][0]), fabsf(raw[sl][1])), fmaxf(fabsf(raw[sl][2]), fabsf(raw[sl][3]))));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // As in matmul_split_x_kernel: mx * 2^-e in [2^12, 2^13), e clamped to [-126, 115].
    int ex = 0;
    if (mx > 0.f && mx <= FLT_MAX) (void)frexpf(mx, &ex);
    const int e = mx > 0.f ? (mx <= FLT_MAX ? min(115, max(-126, ex - 13)) : 115) : 0;
#pragma unroll
    for (int sl = 0; sl < kSlots; ++sl) {
        if (sl * kMmThreads >= n4) break;  // the same for every thread
        const int tt = t + sl * kMmThreads;
        const f4 v = raw[sl] * ldexpf(1.0f, -e);
        if constexpr (kSums) {
            // Eight threads hold a block's 32 values: a tree over the group.
            float s = (v[0] + v[1]) + (v[2] + v[3]);
#pragma unroll
            for (int off = 1; off < 8; off <<= 1) s += __shfl_xor(s, off);
            if (tt < n4 && (tt & 7) == 0) a.xsum[((int64_t)z * 2 * a.chunks_per_split + (tt >> 3)) * 64 + b] = s;
        }
        if (tt < n4) {
            const h4v h = __builtin_convertvector(v, h4v);
            f4 l = v - __builtin_convertvector(h, f4);
#pragma unroll
            for (int c = 0; c < 4; ++c) l[c] = __builtin_isinf(v[c]) ? 0.f : l[c];
            const h4v lh = __builtin_convertvector(l, h4v);
            _Float16* xt = static_cast<_Float16*>(a.xh);
            const int k = 4 * (i0 + tt);
            const int64_t tile0 = (int64_t)(b >> 4) * (a.in_dim / 64);
            const int64_t base = ((tile0 + (k >> 6)) * 2 + ((k >> 5) & 1)) * 2 * 512 +
                                 (((k >> 3) & 3) * 16 + (b & 15)) * 8 + (k & 7);
            *reinterpret_cast<h4v*>(xt + base) = h;
            *reinterpret_cast<h4v*>(xt + base + 512) = lh;
        }
    }
    if (t == 0) a.xexp[z * a.batch + b] = e;
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Eight int8 (two dwords) as fp16: with u = q ^ 0x80, the half 0x6400 | u is
// 1024 + u, so subtracting 1152 leaves q exactly.  v_perm_b32 pairs each byte
// of u with a 0x64 byte from the constant operand.
__device__ __forceinline__ h8 q8_to_h8(uint32_t d0, uint32_t d1) {
    h8 r;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t u = (k ? d1 : d0) ^ 0x80808080u;
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // bytes u0, 64, u1, 64
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes u2, 64, u3, 64
        const h2 a0 = __builtin_bit_cast(h2, p0) - h2{(_Float16)1152.0f, (_Float16)1152.0f};
        const h2 a1 = __builtin_bit_cast(h2, p1) - h2{(_Float16)1152.0f, (_Float16)1152.0f};
        r[4 * k + 0] = a0[0];
        r[4 * k + 1] = a0[1];
        r[4 * k + 2] = a1[0];
        r[4 * k + 3] = a1[1];
    }
    return r;
}

// Four nibbles per dword (one per byte, 0..15) as fp16: the half 0x6400 | q is
// 1024 + q, so subtracting 1024 leaves q exactly.
__device__ __forceinline__ h8 nib_to_h8(uint32_t d0, uint32_t d1) {
    h8 r;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t u = k ? d1 : d0;
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // bytes u0, 64, u1, 64
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes u2, 64, u3, 64
        const h2 a0 = __builtin_bit_cast(h2, p0) - h2{(_Float16)1024.0f, (_Float16)1024.0f};
        const h2 a1 = __builtin_bit_cast(h2, p1) - h2{(_Float16)1024.0f, (_Float16)1024.0f};
        r[4 * k + 0] = a0[0];
        r[4 * k + 1] = a0[1];
        r[4 * k + 2] = a1[0];
        r[4 * k + 3] = a1[1];
    }
    return r;
}

// Four six-bit values (one per byte, 0..63) as fp16 minus 32: the half
// 0x6400 | u is 1024 + u, so subtracting 1056 leaves u - 32 exactly.
__device__ __forceinline__ void six_to_h4(uint32_t u, h2& lo, h2& hi) {
    lo = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - h2{(_Float16)1056.0f, (_Float16)1056.0f};
    hi = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - h2{(_Float16)1056.0f, (_Float16)1056.0f};
}

// The lane's raw words of one 64-wide chunk of its weight row (68 bytes at a
// multiple of 4): block 0's eight values at bytes 2 + 8 g (dwords 2g .. 2g + 2,
// shifted by 2), block 1's at 36 + 8 g (dwords 9 + 2g, 10 + 2g), and the two
// scales (low half of dword 0, high half of dword 8).  All inside the chunk.
struct Q8Raw {
    uint32_t b0[3];
    uint32_t b1[2];
    uint32_t s0, s8;
};

__device__ __forceinline__ void load_q8_raw(Q8Raw& r, const MatmulArgs& a, int o, int c, int g) {
    const int64_t row_bytes = (int64_t)(a.in_dim / 32) * 34;
    const uint32_t* cw =
        reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(a.w) + (int64_t)o * row_bytes + (int64_t)c * 68);
#pragma unroll
    for (int i = 0; i < 3; ++i) r.b0[i] = cw[2 * g + i];
    r.b1[0] = cw[9 + 2 * g];
    r.b1[1] = cw[10 + 2 * g];
    r.s0 = cw[0];
    r.s8 = cw[8];
}

// Q4_K: the lane's words of chunk c of its weight row: the super-block head
// (d | dmin << 16 and the three scale words) and the two quant dwords at bytes
// 32 p + 8 g of the chunk's quarter p, whose low nibbles are block 0's values
// 8 g .. 8 g + 7 (sub-block 2 p) and high nibbles block 1's (sub-block 2 p + 1).
struct Q4KRaw {
    uint32_t hdr;
    uint32_t sc[3];
    uint32_t q[2];
};

__device__ __forceinline__ void load_q4k_raw(Q4KRaw& r, const MatmulArgs& a, int o, int c, int g) {
    const int64_t row_bytes = (int64_t)(a.in_dim / 256) * 144;
    const uint32_t* bw = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(a.w) + (int64_t)o * row_bytes +
                                                           (int64_t)(c >> 2) * 144);
    r.hdr = bw[0];
#pragma unroll
    for (int i = 0; i < 3; ++i) r.sc[i] = bw[1 + i];
    r.q[0] = bw[4 + 8 * (c & 3) + 2 * g];
    r.q[1] = bw[5 + 8 * (c & 3) + 2 * g];
}

// Q6_K: the lane's words of chunk c of its weight row (quarters 2 e and 2 e + 1
// of half hn of the super-block, e = c % 2, hn = c % 4 / 2): the low-bit bytes
// 64 hn + 8 g .. and 64 hn + 32 + 8 g .. (nibble e), the high-bit bytes
// 32 hn + 8 g .. (bits 4 e .. 4 e + 3), the four scales 8 hn + 4 e .. and d.
// Super-blocks are 210 bytes, so these are raw buffer loads at 2-byte aligned
// offsets (gfx950 runs with unaligned buffer access), inside the super-block.
struct Q6KRaw {
    uint32_t l0[2], l1[2], h[2];
    uint32_t sc;
    uint16_t d;
};

__device__ __forceinline__ void load_q6k_raw(Q6KRaw& r, __amdgpu_buffer_rsrc_t wr, int row_off, int c, int g) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const int hn = (c >> 1) & 1;
    const int off = row_off + (c >> 2) * 210;
    const u2 l0 = __builtin_amdgcn_raw_buffer_load_b64(wr, off + 64 * hn + 8 * g, 0, 0);
    const u2 l1 = __builtin_amdgcn_raw_buffer_load_b64(wr, off + 64 * hn + 32 + 8 * g, 0, 0);
    const u2 h = __builtin_amdgcn_raw_buffer_load_b64(wr, off + 128 + 32 * hn + 8 * g, 0, 0);
    r.l0[0] = l0[0];
    r.l0[1] = l0[1];
    r.l1[0] = l1[0];
    r.l1[1] = l1[1];
    r.h[0] = h[0];
    r.h[1] = h[1];
    r.sc = __builtin_amdgcn_raw_buffer_load_b32(wr, off + 192 + 8 * hn + 4 * (c & 1), 0, 0);
    r.d = __builtin_amdgcn_raw_buffer_load_b16(wr, off + 208, 0, 0);
}

// matmul_f16_kernel<WT>: Q8_0, Q4_K or Q6_K weights.  For Q4_K a block's values are
// its quants q (exact in fp16) and its scale d1 = d * sc, and the min term
// m1 * sum_k x_k of each block comes from the pre-pass's block sums: per chunk
// and M tile one v_mfma_f32_16x16x4f32 of the sums (A: batch rows x the
// chunk's two blocks, zero in lane groups 2-3) against the lane's m1 values
// (B), into a second accumulator subtracted before the scaling.  For Q6_K a
// block's values are q - 32 (exact in fp16) with a scale d * sc per 16: the
// block runs as two masked pairs of matrix steps (B zero outside lane groups
// 0-1 or 2-3), each half's sum scaled by its own d * sc.
template <int WT>
__global__ __launch_bounds__(kMmThreads, 2) void matmul_f16_kernel(MatmulArgs a) {
    static_assert(WT == kWeightQ8_0 || WT == kWeightQ4_K || WT == kWeightQ6_K, "Q8_0, Q4_K or Q6_K weights");
    constexpr bool kQ4K = WT == kWeightQ4_K;
    constexpr bool kQ6K = WT == kWeightQ6_K;
    // The chunk of x as fp16 pairs: [buffer][hi, lo][64 batch rows][64 halves + 8 padding].
    __shared__ _Float16 xs[2][2][64][72];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 15;  // weight row within the wave's 16 (B column, result column)
    const int g = lane >> 4;
    const int o0 = blockIdx.x * kMmRowsWg + 16 * wave;
    const int b0 = blockIdx.y * 64;
    const int nt = min(4, (a.batch - b0 + 15) >> 4);
    const int o = min(o0 + n, a.out_dim - 1);
    const int chunks = a.in_dim / 64;
    const int c_begin = blockIdx.z * a.chunks_per_split;
    const int c_end = min(chunks, c_begin + a.chunks_per_split);

    // x staging: thread tid moves batch row tid / 4, halves 16 (tid % 4) .. + 15 of hi and lo.
    const int xr = tid >> 2;
    const int xq = tid & 3;
    const int64_t xoff = (int64_t)min(b0 + xr, a.batch - 1) * a.in_dim + 16 * xq;
    const u4* xh_src = reinterpret_cast<const u4*>(static_cast<const _Float16*>(a.xh) + xoff);
    const u4* xl_src = reinterpret_cast<const u4*>(static_cast<const _Float16*>(a.xl) + xoff);
    u4 xreg[4];
    std::conditional_t<kQ4K, Q4KRaw, std::conditional_t<kQ6K, Q6KRaw, Q8Raw>> wraw;
    // Q6_K: the workgroup's weight rows through one descriptor (the lane's row
    // is clamped to out_dim - 1, as for the other types, so it stays inside).
    const int q6_row_bytes = (a.in_dim / 256) * 210;
    const __amdgpu_buffer_rsrc_t q6w = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(a.w) + (int64_t)blockIdx.x * kMmRowsWg * q6_row_bytes),
        (short)0, min(kMmRowsWg, a.out_dim - (int)blockIdx.x * kMmRowsWg) * q6_row_bytes, 0x00020000);
    float xsr[4];  // Q4_K: block sums of the lane's A operands for the min term
    auto load_chunk = [&](int c) {
        xreg[0] = xh_src[8 * c];
        xreg[1] = xh_src[8 * c + 1];
        xreg[2] = xl_src[8 * c];
        xreg[3] = xl_src[8 * c + 1];
        if constexpr (kQ4K) {
            load_q4k_raw(wraw, a, o, c, g);
            // Lane (n, g < 2): batch row b0 + 16 t + n, block 2 c + g.
#pragma unroll
            for (int t = 0; t < 4; ++t)
                xsr[t] = g < 2 && t < nt ? a.xsum[(int64_t)min(b0 + 16 * t + n, a.batch - 1) * (a.in_dim / 32) + 2 * c + g]
                                         : 0.f;
        } else if constexpr (kQ6K) {
            load_q6k_raw(wraw, q6w, (o - (int)blockIdx.x * kMmRowsWg) * q6_row_bytes, c, g);
        } else {
            load_q8_raw(wraw, a, o, c, g);
        }
    };
    auto store_x = [&](int buf) {
        *reinterpret_cast<u4*>(&xs[buf][0][xr][16 * xq]) = xreg[0];
        *reinterpret_cast<u4*>(&xs[buf][0][xr][16 * xq + 8]) = xreg[1];
        *reinterpret_cast<u4*>(&xs[buf][1][xr][16 * xq]) = xreg[2];
        *reinterpret_cast<u4*>(&xs[buf][1][xr][16 * xq + 8]) = xreg[3];
    };

    f4 acc[4], accm[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = accm[t] = f4{0.f, 0.f, 0.f, 0.f};
    if (c_begin < c_end) {
        load_chunk(c_begin);
        store_x(0);
    }
    __syncthreads();
    for (int c = c_begin; c < c_end; ++c) {
        const int buf = (c - c_begin) & 1;
        // This chunk's two blocks of the lane's row: values and scales.
        h8 wq0, wq1;
        float d0, d1, mb = 0.f, xsc[4];
        float e0 = 0.f, e1 = 0.f;  // Q6_K: the blocks' scales for k >= 16 (d0, d1 for k < 16)
        if constexpr (kQ6K) {
            const int e = c & 1;
            const float d = (float)__builtin_bit_cast(_Float16, wraw.d);
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
                const uint32_t u0 = ((wraw.l0[t2] >> (4 * e)) & 0x0F0F0F0Fu) | (((wraw.h[t2] >> (4 * e)) & 0x03030303u) << 4);
                const uint32_t u1 =
                    ((wraw.l1[t2] >> (4 * e)) & 0x0F0F0F0Fu) | (((wraw.h[t2] >> (4 * e + 2)) & 0x03030303u) << 4);
                h2 lo, hi;
                six_to_h4(u0, lo, hi);
                wq0[4 * t2 + 0] = lo[0];
                wq0[4 * t2 + 1] = lo[1];
                wq0[4 * t2 + 2] = hi[0];
                wq0[4 * t2 + 3] = hi[1];
                six_to_h4(u1, lo, hi);
                wq1[4 * t2 + 0] = lo[0];
                wq1[4 * t2 + 1] = lo[1];
                wq1[4 * t2 + 2] = hi[0];
                wq1[4 * t2 + 3] = hi[1];
            }
            d0 = d * (float)(int8_t)(wraw.sc & 0xFFu);  // exact
            e0 = d * (float)(int8_t)((wraw.sc >> 8) & 0xFFu);
            d1 = d * (float)(int8_t)((wraw.sc >> 16) & 0xFFu);
            e1 = d * (float)(int8_t)(wraw.sc >> 24);
        } else if constexpr (kQ4K) {
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(wraw.hdr & 0xFFFFu));
            const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(wraw.hdr >> 16));
            uint32_t sc0, m0, sc1, m1;
            q4k_scale_min(wraw.sc, 2 * (c & 3), sc0, m0);
            q4k_scale_min(wraw.sc, 2 * (c & 3) + 1, sc1, m1);
            d0 = d * (float)sc0;  // exact
            d1 = d * (float)sc1;
            mb = g == 0 ? dmin * (float)m0 : g == 1 ? dmin * (float)m1 : 0.f;  // B of the min term
            wq0 = nib_to_h8(wraw.q[0] & 0x0F0F0F0Fu, wraw.q[1] & 0x0F0F0F0Fu);
            wq1 = nib_to_h8((wraw.q[0] >> 4) & 0x0F0F0F0Fu, (wraw.q[1] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int t = 0; t < 4; ++t) xsc[t] = xsr[t];
        } else {
            wq0 = q8_to_h8(__builtin_amdgcn_alignbyte(wraw.b0[1], wraw.b0[0], 2),
                           __builtin_amdgcn_alignbyte(wraw.b0[2], wraw.b0[1], 2));
            wq1 = q8_to_h8(wraw.b1[0], wraw.b1[1]);
            d0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(wraw.s0 & 0xFFFFu));
            d1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(wraw.s8 >> 16));
        }
        const bool more = c + 1 < c_end;
        if (more) load_chunk(c + 1);  // the next chunk loads while this one computes
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (t < nt) {
                const int row = 16 * t + n;  // A row: batch row of this lane
#pragma unroll
                for (int blk = 0; blk < 2; ++blk) {
                    const h8 ah = *reinterpret_cast<const h8*>(&xs[buf][0][row][32 * blk + 8 * g]);
                    const h8 al = *reinterpret_cast<const h8*>(&xs[buf][1][row][32 * blk + 8 * g]);
                    const h8 wq = blk ? wq1 : wq0;
                    const float d = blk ? d1 : d0;
                    if constexpr (kQ6K) {
                        const h8 wa = g < 2 ? wq : h8{};  // k < 16 of the block
                        const h8 wb = g < 2 ? h8{} : wq;
                        f4 pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, wa, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, wa, pa, 0, 0, 0);
                        f4 pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, wb, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, wb, pb, 0, 0, 0);
                        const float de = blk ? e1 : e0;
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(de, pb[r], fmaf(d, pa[r], acc[t][r]));
                    } else {
                        f4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, wq, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        part = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, wq, part, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(d, part[r], acc[t][r]);
                    }
                }
                if constexpr (kQ4K) accm[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xsc[t], mb, accm[t], 0, 0, 0);
            }
        }
        if (more) store_x(buf ^ 1);  // the other buffer's last readers passed the previous barrier
        __syncthreads();
    }

    // Lane holds batch rows b0 + 16 t + 4 g + r of weight row o0 + n.
    const int oo = o0 + n;
    if (oo >= a.out_dim) return;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int b = b0 + 16 * t + 4 * g + r;
            if (t >= nt || b >= a.batch) continue;
            const float v = ldexpf(kQ4K ? acc[t][r] - accm[t][r] : acc[t][r], a.xexp[b]);
            float* dst = a.split_out ? a.split_out + ((int64_t)blockIdx.z * a.batch + b) * a.out_dim
                                     : a.y + (int64_t)b * a.out_dim;
            dst[oo] = v;
        }
    }
}

// ---- Q8_0 weights, batches of up to 64 rows ---------------------------------
//
// matmul_q8_f16_small_kernel<NT, CH, kPasses> is the fp16 form for batches of
// at most 64 rows (NT M tiles of 16), laid out so that nothing waits in line:
//   - x comes from the pre-pass in tile order (matmul_split_x_range_kernel):
//     a wave loads the A operands of its M tile straight into registers, one
//     KB per instruction, every chunk of its range at once, with no LDS and no
//     barrier between chunks;
//   - the workgroup's 64 weight rows over its range of at most CH chunks are
//     expanded to fp16 once, into LDS, with their block scales as floats;
//   - a longer range (kPasses: the merge holds too few ranges for chunks of
//     CH, as for an 18944-wide K at 64 rows) is walked CH chunks at a time
//     through the same LDS, with a barrier between passes;
//   - wave w takes M tile w NT / 4 and NT of the four N tiles (16 weight rows
//     each), so every staged operand serves several matrix steps;
//   - two workgroups fit on a CU;
//   - with K split over grid.z, each workgroup stores its tile coherently,
//     waits for the stores and counts itself on the output tile's counter; the
//     last one adds the ranges' tiles in z order (its own from registers),
//     every load issued before the first add, and resets the counter.  No
//     reduce launch, and results do not depend on timing.
constexpr int kSmMaxPartials = 32;  // K ranges x tiles per lane the merge holds at most
constexpr int kSmRowHalves = 8 * 64 + 8;  // an LDS weight row: 8 chunks of 64 halves, +16 bytes

// The small forms' shared steps.  Wave w of a workgroup takes M tile
// mt = w NT / 4 (batch rows 16 mt ..) against N tiles nt0 .. nt0 + NT - 1
// (weight rows 64 blockIdx.x + 16 nt0 ..); lane (g = lane / 16, n = lane % 16).

// A operands of the wave's M tile, every chunk of the range at once:
// [chunk][block][hi, lo], one KB per load from the pre-pass's tile order.
template <int CH>
__device__ __forceinline__ void small_load_x(h8 (&ax)[CH][2][2], const MatmulArgs& a, int mt, int chunks, int c_begin,
                                             int nc, int lane) {
    const h8* xt = reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.xh)) +
                   ((int64_t)mt * chunks + c_begin) * 256 + lane;
#pragma unroll
    for (int i = 0; i < CH; ++i)
        if (i < nc)
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
                for (int part = 0; part < 2; ++part) ax[i][blk][part] = xt[i * 256 + (blk * 2 + part) * 64];
}

// One pass's products: per block, hi and lo into a fresh accumulator, which
// the block's scale (wd: [weight row][2 chunk + block]) adds into acc.
template <int NT, int CH>
__device__ __forceinline__ void small_products(f4 (&acc)[NT], const h8 (&ax)[CH][2][2], const _Float16* wh,
                                               const float (*wd)[2 * CH + 1], int nc, int nt0, int n, int g) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        if (i < nc) {
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int r = 16 * (nt0 + j) + n;  // B column: the lane's weight row
                    const h8 wq = *reinterpret_cast<const h8*>(&wh[r * kSmRowHalves + i * 64 + blk * 32 + g * 8]);
                    const float d = wd[r][2 * i + blk];
                    f4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[i][blk][0], wq, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    part = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[i][blk][1], wq, part, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[j][q] = fmaf(d, part[q], acc[j][q]);
                }
            }
        }
    }
}

// The tile's end: scale by 2^xexp of each batch row's K range, then either
// store y (one range) or store the partial coherently, count the tile and, in
// the last workgroup of the tile, add the ranges in z order (every load issued
// before the first add) and reset the counter.
template <int NT>
__device__ __forceinline__ void small_finish(const MatmulArgs& a, const f4 (&acc)[NT], int mt, int nt0, int n, int g,
                                             int tid, int& last) {
    // Lane holds batch rows 16 mt + 4 g + q of weight rows 64 x + 16 (nt0 + j) + n,
    // scaled by 2^-xexp of the batch row's K range.
    float v[NT][4];
    int bq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bq[q] = 16 * mt + 4 * g + q;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = a.xexp[blockIdx.z * a.batch + min(bq[q], a.batch - 1)];
#pragma unroll
        for (int j = 0; j < NT; ++j) v[j][q] = ldexpf(acc[j][q], e);
    }
    const int obase = blockIdx.x * kMmRowsWg + 16 * nt0 + n;
    if (a.splits == 1) {
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (obase + 16 * j < a.out_dim && bq[q] < a.batch) a.y[(int64_t)bq[q] * a.out_dim + obase + 16 * j] = v[j][q];
        return;
    }
    const int z = blockIdx.z;
    const int64_t plane = (int64_t)a.batch * a.out_dim;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (obase + 16 * j < a.out_dim && bq[q] < a.batch)
                coherent_store(a.split_out + z * plane + (int64_t)bq[q] * a.out_dim + obase + 16 * j, v[j][q]);
    wait_vm_complete();
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(a.counters + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               a.splits - 1;
    __syncthreads();
    if (!last) return;
    constexpr int kZ = kSmMaxPartials / NT;
    float p[NT][4][kZ];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float* pb = a.split_out + (int64_t)min(bq[q], a.batch - 1) * a.out_dim + min(obase + 16 * j, a.out_dim - 1);
#pragma unroll
            for (int zz = 0; zz < kZ; ++zz) p[j][q][zz] = coherent_load(pb + min(zz, a.splits - 1) * plane);
        }
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float s = z == 0 ? v[j][q] : p[j][q][0];
#pragma unroll
            for (int zz = 1; zz < kZ; ++zz)
                if (zz < a.splits) s += zz == z ? v[j][q] : p[j][q][zz];
            if (obase + 16 * j < a.out_dim && bq[q] < a.batch) a.y[(int64_t)bq[q] * a.out_dim + obase + 16 * j] = s;
        }
    if (tid == 0) __hip_atomic_store(a.counters + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int NT, int CH, bool kPasses>
__global__ __launch_bounds__(kMmThreads, 2) void matmul_q8_f16_small_kernel(MatmulArgs a) {
    static_assert(CH <= 8, "an LDS weight row holds 8 chunks");
    __shared__ _Float16 wh[kMmRowsWg * kSmRowHalves];  // [weight row][chunk][64 halves]
    __shared__ float wd[kMmRowsWg][2 * CH + 1];        // block scales [weight row][2 chunk + block]
    __shared__ int last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int chunks = a.in_dim / 64;
    const int c_begin = blockIdx.z * a.chunks_per_split;
    const int nc_range = min(chunks, c_begin + a.chunks_per_split) - c_begin;  // 1..CH, or more with kPasses (host)
    constexpr int kWavesPerM = 4 / NT;
    const int mt = wave / kWavesPerM;           // the wave's M tile
    const int nt0 = (wave % kWavesPerM) * NT;   // its first N tile

    f4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f4{0.f, 0.f, 0.f, 0.f};
    // With kPasses the range is walked CH chunks at a time through the same LDS.
    for (int c0 = 0;;) {
        const int nc = kPasses ? min(CH, nc_range - c0) : nc_range;
        const int cb = c_begin + c0;
        h8 ax[CH][2][2];
        small_load_x<CH>(ax, a, mt, chunks, cb, nc, lane);

        // Weights to fp16: unit u = 64 r + 8 i + 4 block + gg (row r, chunk i, lane
        // group gg) is eight values; thread tid takes units tid + 256 k, that is
        // one fixed (chunk, block, lane group) of rows tid / 64 + 4 k.  A wave's
        // units are one row's chunks, so its loads cover whole 68-byte windows.
        // Every unit's three dwords load first, one 12-byte raw buffer load each
        // (dword aligned; one lane offset per thread): block 0's values sit at
        // dwords 2 gg .. 2 gg + 2 shifted by 2 bytes, block 1's at 9 + 2 gg,
        // 10 + 2 gg (the load covers 8 + 2 gg .. 10 + 2 gg), and the scale is the
        // low half of dword 0 or the high half of dword 8, both in lane group 0's
        // load.
        // Units of chunks past the range load the range's last chunk and store
        // nothing; rows past out_dim read as zero (past the buffer's end).
        {
            constexpr int kU = (kMmRowsWg * 64) / kMmThreads;
            const int row_bytes = chunks * 68;
            const int rows_here = min(kMmRowsWg, a.out_dim - (int)blockIdx.x * kMmRowsWg);
            typedef uint32_t u3 __attribute__((ext_vector_type(3)));
            const int r0 = tid >> 6;
            const int i = (tid >> 3) & 7;
            const int blk = (tid >> 2) & 1;
            const int gg = tid & 3;
            const int s0 = blk ? 8 + 2 * gg : 2 * gg;  // the unit's three dwords: s0 .. s0 + 2, inside the chunk
            const int voff = r0 * row_bytes + (cb + min(i, nc - 1)) * 68 + 4 * s0;
            u3 wdw[kU];
#pragma unroll
            for (int k = 0; k < kU; ++k) {
                // Rows r0 + 4 k: the row step goes into the descriptor (base and
                // record count), so one lane offset serves every load and the
                // range check, which covers the lane offset, still stops at out_dim.
                const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<uint8_t*>(static_cast<const uint8_t*>(a.w) + ((int64_t)blockIdx.x * kMmRowsWg + 4 * k) * row_bytes),
                    (short)0, max(0, rows_here - 4 * k) * row_bytes, 0x00020000);
                wdw[k] = __builtin_amdgcn_raw_buffer_load_b96(wr, voff, 0, 0);
            }
            const int sh = blk ? 0 : 2;
            _Float16* wdst = &wh[r0 * kSmRowHalves + i * 64 + blk * 32 + gg * 8];
            float* ddst = &wd[r0][2 * i + blk];
            if (i < nc) {
#pragma unroll
                for (int k = 0; k < kU; ++k) {
                    const uint32_t d0 = blk ? wdw[k][1] : wdw[k][0];
                    const uint32_t d1 = blk ? wdw[k][2] : wdw[k][1];
                    const h8 q = q8_to_h8(__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(wdw[k][2], d1, sh));
                    *reinterpret_cast<h8*>(wdst + 4 * k * kSmRowHalves) = q;
                    // Lane group 0 holds the block's scale: dword 0 (low half) or 8 (high half).
                    const uint32_t sw = blk ? wdw[k][0] >> 16 : wdw[k][0];
                    if (gg == 0) ddst[4 * k * (2 * CH + 1)] = (float)__builtin_bit_cast(_Float16, (uint16_t)(sw & 0xFFFFu));
                }
            }
        }
        __syncthreads();

        small_products<NT, CH>(acc, ax, wh, wd, nc, nt0, n, g);
        if constexpr (!kPasses) break;
        c0 += CH;
        if (c0 >= nc_range) break;
        __syncthreads();  // every wave is done with this pass's weights
    }
    small_finish<NT>(a, acc, mt, nt0, n, g, tid, last);
}

// ---- Q4_K weights, batches of up to 64 rows ---------------------------------
//
// matmul_q4k_f16_small_kernel<NT, kPasses> is the Q8_0 small form with Q4_K weights.
// A weight is w = d1 q - m1 per 32-wide sub-block (d1 = d * sc and
// m1 = dmin * m, both exact in fp32; q = 0..15, exact in fp16), so
//   y[b][o] = sum over blocks of  d1 * sum_k q_k x_k  -  m1 * sum_k x_k.
// The first term is the Q8_0 form's: the quants go to LDS as fp16 and each
// block is one hi/lo pair of 16x16x32 fp16 matrix steps scaled by d1.  The
// second needs only the blocks' sums of x, which the pre-pass writes (of the
// scaled x, so both terms carry the range's 2^-xexp): per four blocks one
// v_mfma_f32_16x16x4f32 of the x sums (A: batch rows x blocks) against the
// m1 values (B: blocks x weight rows) into a second accumulator, subtracted
// before the scaling.  A chunk of 64 weights is one quarter p of a 256-weight
// super-block: sub-blocks 2 p (low nibbles of quant bytes 32 p ..) and 2 p + 1
// (their high nibbles), so ranges need not start on a super-block.
template <int NT, bool kPasses>
__global__ __launch_bounds__(kMmThreads, 2) void matmul_q4k_f16_small_kernel(MatmulArgs a) {
    constexpr int CH = 8;
    __shared__ _Float16 wh[kMmRowsWg * kSmRowHalves];  // quants [weight row][chunk][64 halves]
    __shared__ float wd[kMmRowsWg][2 * CH + 1];        // d1 = d * sc [weight row][2 chunk + block]
    __shared__ float wm[kMmRowsWg][2 * CH + 1];        // m1 = dmin * m, the same way
    __shared__ __attribute__((aligned(16))) float xs[2 * CH][64];  // block sums of scaled x [block][batch row]
    __shared__ int last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int chunks = a.in_dim / 64;
    const int c_begin = blockIdx.z * a.chunks_per_split;
    const int nc_range = min(chunks, c_begin + a.chunks_per_split) - c_begin;  // 1..CH, or more with kPasses (host)
    constexpr int kWavesPerM = 4 / NT;
    const int mt = wave / kWavesPerM;
    const int nt0 = (wave % kWavesPerM) * NT;

    f4 acc[NT], accm[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = accm[j] = f4{0.f, 0.f, 0.f, 0.f};
    // With kPasses the range is walked CH chunks at a time through the same LDS.
    for (int c0 = 0;;) {
        const int nc = kPasses ? min(CH, nc_range - c0) : nc_range;
        const int cb = c_begin + c0;
        h8 ax[CH][2][2];
        small_load_x<CH>(ax, a, mt, chunks, cb, nc, lane);

        // Weights: unit (row r, chunk i) is one super-block quarter, 64 quants in 32
        // bytes plus the super-block's 16-byte head (d, dmin, the 12 scale bytes);
        // thread tid takes chunk tid % 8 of rows tid / 8 and tid / 8 + 32, three
        // 16-byte raw buffer loads each (super-blocks are 144 bytes, so every load
        // is dword aligned), all issued before the first is used.  Units of chunks
        // past the range load the range's last chunk and store zero scales; rows
        // past out_dim read as zero (past the buffer's end).
        {
            const int row_bytes = (a.in_dim / 256) * 144;
            const int rows_here = min(kMmRowsWg, a.out_dim - (int)blockIdx.x * kMmRowsWg);
            const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint8_t*>(static_cast<const uint8_t*>(a.w) + (int64_t)blockIdx.x * kMmRowsWg * row_bytes),
                (short)0, rows_here * row_bytes, 0x00020000);
            const int i = tid & 7;
            const int r0 = tid >> 3;
            const int c = cb + min(i, nc - 1);
            const int p = c & 3;
            const int voff = r0 * row_bytes + (c >> 2) * 144;
            u4 hd[2], qa[2], qb[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int off = voff + 32 * k * row_bytes;
                hd[k] = __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0);
                qa[k] = __builtin_amdgcn_raw_buffer_load_b128(wr, off + 16 + 32 * p, 0, 0);
                qb[k] = __builtin_amdgcn_raw_buffer_load_b128(wr, off + 32 + 32 * p, 0, 0);
            }
            // The range's block sums, loaded after the weights (the memory counter
            // drains in order, so the weights need not wait for them) and stored
            // after the expansion: thread tid takes block tid / 16, batch rows
            // 4 (tid % 16) .. + 3; blocks past the range and rows past the batch are 0.
            const int sblk = tid >> 4;
            const int b4 = 4 * (tid & 15);
            f4 xsv = f4{0.f, 0.f, 0.f, 0.f};
            if (sblk < 2 * nc)
                xsv = *reinterpret_cast<const f4*>(a.xsum + ((int64_t)blockIdx.z * 2 * a.chunks_per_split + 2 * c0 + sblk) * 64 + b4);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int r = r0 + 32 * k;
                float d1[2] = {0.f, 0.f}, m1[2] = {0.f, 0.f};
                if (i < nc) {
                    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd[k][0] & 0xFFFFu));
                    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hd[k][0] >> 16));
                    const uint32_t sc[3] = {hd[k][1], hd[k][2], hd[k][3]};
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        uint32_t scv, mv;
                        q4k_scale_min(sc, 2 * p + h, scv, mv);
                        d1[h] = d * (float)scv;   // exact
                        m1[h] = dmin * (float)mv;  // exact
                    }
                    const uint32_t q[8] = {qa[k][0], qa[k][1], qa[k][2], qa[k][3], qb[k][0], qb[k][1], qb[k][2], qb[k][3]};
                    _Float16* dst = &wh[r * kSmRowHalves + i * 64];
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        *reinterpret_cast<h8*>(dst + 8 * s) = nib_to_h8(q[2 * s] & 0x0F0F0F0Fu, q[2 * s + 1] & 0x0F0F0F0Fu);
                        *reinterpret_cast<h8*>(dst + 32 + 8 * s) =
                            nib_to_h8((q[2 * s] >> 4) & 0x0F0F0F0Fu, (q[2 * s + 1] >> 4) & 0x0F0F0F0Fu);
                    }
                }
                wd[r][2 * i] = d1[0];
                wd[r][2 * i + 1] = d1[1];
                wm[r][2 * i] = m1[0];
                wm[r][2 * i + 1] = m1[1];
            }
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (b4 + c >= a.batch) xsv[c] = 0.f;
            *reinterpret_cast<f4*>(&xs[sblk][b4]) = xsv;
        }
        __syncthreads();

        small_products<NT, CH>(acc, ax, wh, wd, nc, nt0, n, g);
        // The min term, four blocks per matrix step: lane (g, n) supplies block
        // 4 s + g of batch row 16 mt + n (A) and of weight row 16 (nt0 + j) + n (B).
#pragma unroll
        for (int s = 0; s < CH / 2; ++s) {
            if (2 * s < nc) {
                const float xa = xs[4 * s + g][16 * mt + n];
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    accm[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, wm[16 * (nt0 + j) + n][4 * s + g], accm[j], 0, 0, 0);
            }
        }
        if constexpr (!kPasses) break;
        c0 += CH;
        if (c0 >= nc_range) break;
        __syncthreads();  // every wave is done with this pass's weights and sums
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] -= accm[j];
    small_finish<NT>(a, acc, mt, nt0, n, g, tid, last);
}

// ---- Q6_K weights, batches of up to 64 rows ---------------------------------
//
// matmul_q6k_f16_small_kernel<NT, kPasses> is the Q8_0 small form with Q6_K
// weights.  A weight is w = (d * sc) * (q - 32) with the int8 scale sc per 16
// weights: q - 32 is exact in fp16 and d * sc exact in fp32, but the scale
// changes inside a 32-wide matrix step.  So each block runs as two masked
// pairs of 16x16x32 fp16 steps (B operand zero outside the lanes of one
// 16-wide half: lane groups 0-1 hold k < 16, 2-3 the rest), each half's sum
// scaled by its own d * sc.  The unit of staging is one 128-weight half n of a
// super-block (chunks 2 n' and 2 n' + 1 of the range, so ranges start on even
// chunks): quant bytes 64 n .. (low 4 bits, the chunk's nibble), high-bit
// bytes 128 + 32 n .., scales 192 + 8 n .. and d at 208.  Super-blocks are
// 210 bytes, so the loads are only 2-byte aligned; gfx950 runs with unaligned
// buffer access, and every load stays inside its super-block.
template <int NT, int CH>
__device__ __forceinline__ void small_products_q6k(f4 (&acc)[NT], const h8 (&ax)[CH][2][2], const _Float16* wh,
                                                   const float (*ws)[4 * CH + 1], int nc, int nt0, int n, int g) {
    const h8 zero = h8{};
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        if (i < nc) {
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int r = 16 * (nt0 + j) + n;
                    const h8 wq = *reinterpret_cast<const h8*>(&wh[r * kSmRowHalves + i * 64 + blk * 32 + g * 8]);
                    const h8 wa = g < 2 ? wq : zero;  // k < 16: the block's first scale
                    const h8 wb = g < 2 ? zero : wq;
                    const float sa = ws[r][4 * i + 2 * blk];
                    const float sb = ws[r][4 * i + 2 * blk + 1];
                    f4 pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[i][blk][0], wa, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[i][blk][1], wa, pa, 0, 0, 0);
                    f4 pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[i][blk][0], wb, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[i][blk][1], wb, pb, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[j][q] = fmaf(sb, pb[q], fmaf(sa, pa[q], acc[j][q]));
                }
            }
        }
    }
}

template <int NT, bool kPasses>
__global__ __launch_bounds__(kMmThreads, 2) void matmul_q6k_f16_small_kernel(MatmulArgs a) {
    constexpr int CH = 8;
    __shared__ _Float16 wh[kMmRowsWg * kSmRowHalves];  // q - 32 [weight row][chunk][64 halves]
    __shared__ float ws[kMmRowsWg][4 * CH + 1];        // d * sc [weight row][4 chunk + 16-wide part]
    __shared__ int last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int chunks = a.in_dim / 64;
    const int c_begin = blockIdx.z * a.chunks_per_split;  // even (host)
    const int nc_range = min(chunks, c_begin + a.chunks_per_split) - c_begin;  // 1..CH, or more with kPasses (host)
    constexpr int kWavesPerM = 4 / NT;
    const int mt = wave / kWavesPerM;
    const int nt0 = (wave % kWavesPerM) * NT;

    // Staging: thread tid takes row tid / 4 and the range's half tid % 4 (its
    // chunks 2 (tid % 4) and 2 (tid % 4) + 1); a wave's loads cover 16 rows.
    const int row_bytes = (a.in_dim / 256) * 210;
    const int rows_here = min(kMmRowsWg, a.out_dim - (int)blockIdx.x * kMmRowsWg);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(a.w) + (int64_t)blockIdx.x * kMmRowsWg * row_bytes), (short)0,
        rows_here * row_bytes, 0x00020000);
    const int r = tid >> 2;
    const int hh = tid & 3;

    f4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f4{0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0;;) {
        const int nc = kPasses ? min(CH, nc_range - c0) : nc_range;
        const int cb = c_begin + c0;
        h8 ax[CH][2][2];
        small_load_x<CH>(ax, a, mt, chunks, cb, nc, lane);
        {
            // The unit's half of the super-block (the range's last when past it).
            const int hl = min(2 * hh, nc - 1) >> 1;
            const int half = (cb >> 1) + hl;
            const int hn = half & 1;
            const int off = r * row_bytes + (half >> 1) * 210;
            u4 ql[4], qh[2];
#pragma unroll
            for (int t = 0; t < 4; ++t) ql[t] = __builtin_amdgcn_raw_buffer_load_b128(wr, off + 64 * hn + 16 * t, 0, 0);
#pragma unroll
            for (int t = 0; t < 2; ++t) qh[t] = __builtin_amdgcn_raw_buffer_load_b128(wr, off + 128 + 32 * hn + 16 * t, 0, 0);
            typedef uint32_t u2 __attribute__((ext_vector_type(2)));
            const u2 sc = __builtin_amdgcn_raw_buffer_load_b64(wr, off + 192 + 8 * hn, 0, 0);
            const uint16_t dh = __builtin_amdgcn_raw_buffer_load_b16(wr, off + 208, 0, 0);
            const float d = (float)__builtin_bit_cast(_Float16, dh);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int i = 2 * hh + e;  // the chunk in this pass
                if (i < nc) {
                    _Float16* dst = &wh[r * kSmRowHalves + i * 64];
#pragma unroll
                    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
                        for (int s = 0; s < 4; ++s) {
                            h8 v;
#pragma unroll
                            for (int t2 = 0; t2 < 2; ++t2) {
                                const int t = 2 * s + t2;  // dword of the block: its weights 4 t .. 4 t + 3
                                const uint32_t qlw = ql[(8 * blk + t) >> 2][(8 * blk + t) & 3];
                                const uint32_t qhw = qh[t >> 2][t & 3];
                                const uint32_t u = ((qlw >> (4 * e)) & 0x0F0F0F0Fu) |
                                                   (((qhw >> (4 * e + 2 * blk)) & 0x03030303u) << 4);
                                h2 lo, hi;
                                six_to_h4(u, lo, hi);
                                v[4 * t2 + 0] = lo[0];
                                v[4 * t2 + 1] = lo[1];
                                v[4 * t2 + 2] = hi[0];
                                v[4 * t2 + 3] = hi[1];
                            }
                            *reinterpret_cast<h8*>(dst + blk * 32 + 8 * s) = v;
                        }
                    }
                    // Scales 8 hn + 4 e + 2 blk + part: byte 2 blk + part of scale dword e.
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        ws[r][4 * i + p] = d * (float)(int8_t)((sc[e] >> (8 * p)) & 0xFFu);  // exact
                }
            }
        }
        __syncthreads();
        small_products_q6k<NT, CH>(acc, ax, wh, ws, nc, nt0, n, g);
        if constexpr (!kPasses) break;
        c0 += CH;
        if (c0 >= nc_range) break;
        __syncthreads();  // every wave is done with this pass's weights
    }
    small_finish<NT>(a, acc, mt, nt0, n, g, tid, last);
}

// y = the sum over z of the split partials, in z order; four elements per
// thread and step when y and the partials are 16-byte aligned, else one.
__global__ __launch_bounds__(kMmThreads) void matmul_reduce_kernel(MatmulArgs a) {
    const int64_t n = (int64_t)a.batch * a.out_dim;
    const int64_t stride = (int64_t)gridDim.x * kMmThreads;
    const int64_t first = (int64_t)blockIdx.x * kMmThreads + threadIdx.x;
    if (n % 4 == 0 && reinterpret_cast<uintptr_t>(a.y) % 16 == 0) {
        const f4* src = reinterpret_cast<const f4*>(a.split_out);
        f4* dst = reinterpret_cast<f4*>(a.y);
        const int64_t n4 = n / 4;
        for (int64_t i = first; i < n4; i += stride) {
            f4 s = src[i];
            for (int z = 1; z < a.splits; ++z) s += src[(int64_t)z * n4 + i];
            dst[i] = s;
        }
        return;
    }
    for (int64_t i = first; i < n; i += stride) {
        float s = a.split_out[i];
        for (int z = 1; z < a.splits; ++z) s += a.split_out[(int64_t)z * n + i];
        a.y[i] = s;
    }
}

}  // namespace

int matmul_small_chunks(int) { return 8; }

int matmul_small_range_chunks_max() { return 4 * kMmThreads / 16; }  // the pre-pass: four f4 per thread

int64_t matmul_small_x_halves(int batch, int in_dim) {
    return (int64_t)(batch <= 16 ? 1 : batch <= 32 ? 2 : 4) * 16 * in_dim * 2;  // NT whole M tiles, hi and lo
}

int matmul_small_max_splits(int batch) { return kSmMaxPartials / (batch <= 16 ? 1 : batch <= 32 ? 2 : 4); }

namespace {

template <int NT, bool kPasses>
void launch_small_product(const MatmulArgs& a, dim3 grid, hipStream_t stream) {
    if (a.w_type == kWeightQ4_K)
        hipLaunchKernelGGL((matmul_q4k_f16_small_kernel<NT, kPasses>), grid, dim3(kMmThreads), 0, stream, a);
    else if (a.w_type == kWeightQ6_K)
        hipLaunchKernelGGL((matmul_q6k_f16_small_kernel<NT, kPasses>), grid, dim3(kMmThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((matmul_q8_f16_small_kernel<NT, 8, kPasses>), grid, dim3(kMmThreads), 0, stream, a);
}

template <bool kPasses>
void launch_small_product(const MatmulArgs& a, dim3 grid, hipStream_t stream) {
    if (a.batch <= 16)
        launch_small_product<1, kPasses>(a, grid, stream);
    else if (a.batch <= 32)
        launch_small_product<2, kPasses>(a, grid, stream);
    else
        launch_small_product<4, kPasses>(a, grid, stream);
}

}  // namespace

hipError_t launch_matmul_small(const MatmulArgs& a, hipStream_t stream) {
    if (a.batch <= 0 || a.out_dim <= 0) return hipSuccess;
    const bool q4k = a.w_type == kWeightQ4_K;
    const bool q6k = a.w_type == kWeightQ6_K;
    if (a.batch > 64 || (a.w_type != kWeightQ8_0 && !q4k && !q6k) || !a.xh || !a.xl || !a.xexp ||
        a.chunks_per_split < 1 || a.chunks_per_split > matmul_small_range_chunks_max() ||
        a.splits > matmul_small_max_splits(a.batch) || (a.splits > 1 && (!a.split_out || !a.counters)) ||
        (q4k && (!a.xsum || a.in_dim % 256 != 0)) || (q6k && (a.in_dim % 256 != 0 || a.chunks_per_split % 2 != 0)))
        return hipErrorInvalidValue;
    const dim3 pre(a.batch, a.splits);
    if (a.chunks_per_split * 16 <= kMmThreads) {
        if (q4k)
            hipLaunchKernelGGL((matmul_split_x_range_kernel<true, 1>), pre, dim3(kMmThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((matmul_split_x_range_kernel<false, 1>), pre, dim3(kMmThreads), 0, stream, a);
    } else {
        if (q4k)
            hipLaunchKernelGGL((matmul_split_x_range_kernel<true, 4>), pre, dim3(kMmThreads), 0, stream, a);
        else
            hipLaunchKernelGGL((matmul_split_x_range_kernel<false, 4>), pre, dim3(kMmThreads), 0, stream, a);
    }
    const dim3 grid((a.out_dim + kMmRowsWg - 1) / kMmRowsWg, 1, a.splits);
    if (a.chunks_per_split <= matmul_small_chunks(a.batch))
        launch_small_product<false>(a, grid, stream);
    else
        launch_small_product<true>(a, grid, stream);
    return hipGetLastError();
}

hipError_t launch_matmul(const MatmulArgs& a, hipStream_t stream) {
    if (a.batch <= 0 || a.out_dim <= 0) return hipSuccess;
    const dim3 grid((a.out_dim + kMmRowsWg - 1) / kMmRowsWg, (a.batch + 63) / 64, a.splits);
    if (a.w_type == kWeightF32)
        hipLaunchKernelGGL(matmul_batch_kernel<kWeightF32>, grid, dim3(kMmThreads), 0, stream, a);
    else if (a.w_type == kWeightQ8_0 && a.xh) {
        hipLaunchKernelGGL(matmul_split_x_kernel<false>, dim3(a.batch), dim3(kMmThreads), 0, stream, a);
        hipLaunchKernelGGL(matmul_f16_kernel<kWeightQ8_0>, grid, dim3(kMmThreads), 0, stream, a);
    } else if (a.w_type == kWeightQ4_K && a.xh && a.xsum && a.in_dim % 256 == 0) {
        hipLaunchKernelGGL(matmul_split_x_kernel<true>, dim3(a.batch), dim3(kMmThreads), 0, stream, a);
        hipLaunchKernelGGL(matmul_f16_kernel<kWeightQ4_K>, grid, dim3(kMmThreads), 0, stream, a);
    } else if (a.w_type == kWeightQ6_K && a.xh && a.in_dim % 256 == 0) {
        hipLaunchKernelGGL(matmul_split_x_kernel<false>, dim3(a.batch), dim3(kMmThreads), 0, stream, a);
        hipLaunchKernelGGL(matmul_f16_kernel<kWeightQ6_K>, grid, dim3(kMmThreads), 0, stream, a);
    } else if (a.w_type == kWeightQ8_0)
        hipLaunchKernelGGL(matmul_batch_kernel<kWeightQ8_0>, grid, dim3(kMmThreads), 0, stream, a);
    else if (a.w_type == kWeightQ4_K && a.in_dim % 256 == 0)
        hipLaunchKernelGGL(matmul_batch_kernel<kWeightQ4_K>, grid, dim3(kMmThreads), 0, stream, a);
    else if (a.w_type == kWeightQ6_K && a.in_dim % 256 == 0)
        hipLaunchKernelGGL(matmul_batch_kernel<kWeightQ6_K>, grid, dim3(kMmThreads), 0, stream, a);
    else
        return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splits <= 1) return e;
    const int64_t n = (int64_t)a.batch * a.out_dim;
    const int blocks = (int)std::min<int64_t>((n / 4 + kMmThreads - 1) / kMmThreads + 1, 2048);
    hipLaunchKernelGGL(matmul_reduce_kernel, dim3(blocks), dim3(kMmThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace gsp
