// Matrix-core (MFMA) decode of the paged-attention step, gfx950: the device
// code of paged_decode_mfma_kernel (gsp_decode_mfma.hip), which the mixed-step
// kernel (gsp_prefill_mfma.hip) runs too.
//
// Same contract as the DPP decode kernel (PagedAttentionKernel.cs:17-372 over
// every query token of a packed step), but the GQA group turns each 16-token
// page into two small dense contractions that run on the matrix cores:
//
//   S^T[token][head] = K_page[16 x d] . (Q_group * scale * log2 e)^T   (v_mfma_f32_16x16x4f32, M = tokens, N = heads)
//   O[head][e]      += P[16 heads x 16 tokens] . V_page[16 x d]          (v_mfma_f32_16x16x4f32, M = heads, K = tokens)
//
// Heads of the group beyond G are zero padding (G <= 16).  MFMA operand
// layouts for fp32 pages (lane l, n = l % 16, g = l / 16):
//   QK step kk = 4j + i uses d = 16j + 4g + i:  A = K[token n][d],  B = Q[head n][d]
//   result: lane holds S[head n][token 4g + r], r = 0..3
//   PV step kk uses token 4g + kk:  A = P[head n][token 4g + kk] (the lane's own r = kk),
//   B = V[token 4g + kk][e], e = 64c + 4n + i for output block 4c + i
//   result: lane holds O[head 4g + r][e].
// fp16 pages run the same contractions on v_mfma_f32_16x16x16f16 from the
// same registers (one rank-16 step covers d = 16j + 4g + 0..3, or tokens
// 4g + 0..3): K and V are exact in fp16, Q and P enter as hi + lo fp16 pairs,
// accumulation is fp32.  So each lane reads 16-byte (8-byte for fp16) pieces
// of K rows and V rows straight into MFMA operands; the softmax needs one
// max-reduction across the four lane groups per page and four exp2 per lane.
// Page loads are raw buffer loads whose descriptor covers only the page's
// valid tokens: slots past the context read as zero in hardware (no fetch,
// no NaN from stale slots reaches P.V).  Each wave streams every
// kDecodeWaves-th page of its unit with the next page's loads in flight
// while the current one is computed; the four waves merge through LDS and
// split units merge in the epilogue (gsp_epilogue.h).
//
// Shapes.  The fixed-shape instantiations (kExact) take head_dim ==
// v_head_dim == DP in {64, 128} and 16-token pages, all compile-time.  The
// general ones take any head_dim and v_head_dim up to DP (64, 128 or 256) and
// pages of 1..16 tokens at run time, the domain of the reference GPU runner
// (CudaPagedTransformerRunner.cs:402-412) and of the CPU kernel's generic
// path, which takes odd widths too (PagedAttentionKernel.cs:326-370):
//  - a page of bs < 16 tokens fills the tile's first bs rows; the rest read
//    as zero (past the descriptor's range) and are masked like a short page;
//  - dims past head_dim (v_head_dim) are loaded from an offset past the
//    descriptor's range, so they read as zero without a fetch; Q's are zero,
//    so padded dims add nothing to S, and padded O columns are never stored;
//  - kVec4 loads 4 dims per piece (head_dim, v_head_dim multiples of 4);
//    kVec2 loads 2 (any even widths) and kVec1 one (odd widths, whose rows
//    are not 8-byte aligned), so a piece never straddles a row.
// A GQA group above 16 heads runs as tiles of 16 over grid.y, each tile
// rereading the pages (the reference CPU kernel rereads them per head).
#pragma once

#include "gsp_epilogue.h"

namespace gsp {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

enum DecodeMode { kExact = 0, kVec4 = 1, kVec2 = 2, kVec1 = 3 };

constexpr int kTileTokens = 16;  // token rows of a page tile (MFMA M for S^T)
// An element offset past any page's descriptor range: the load reads zero
// and fetches nothing.
constexpr int kOutOfRange = 1 << 28;

// Widths and page size of a launch: compile-time for kExact, run time otherwise.
// A decode tile is m consecutive pages of bs tokens (tt = m bs <= 16 rows).
template <int DP, int MODE>
struct Geo {
    int d, dv, bs, m, tt;
    __device__ explicit Geo(const DecodeArgs& a)
        : d(a.head_dim), dv(a.v_head_dim), bs(a.block_size), m(a.tile_pages), tt(a.block_size * a.tile_pages) {}
};
template <int DP>
struct Geo<DP, kExact> {
    static constexpr int d = DP, dv = DP, bs = kBlockSize, m = 1, tt = kBlockSize;
    __device__ explicit Geo(const DecodeArgs&) {}
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const void* base, int bytes) {
    // Raw buffer (stride 0) of `bytes` bytes; offsets at or past the end read 0.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// Page operands in registers, as stored in the pool (fp16 pages stay fp16).
//   k[j]     = K[token n][16j + 4g .. +3]
//   v[kk][c] = V[token 4g + kk][64c + 4n .. +3]
template <int D, typename KT>
struct PageRegs;

// Exact-shape fp16 pages take the K = 32 fp16 matrix step for the scores:
// lane (n, g) holds K[key n][32 j + 8 g .. + 7] (one 16-byte load, half a
// 128-byte line of the row) and Q[head n][the same dims].  Other fp16 shapes
// use the K = 16 step with 8-byte pieces at 16 j + 4 g.
template <typename KT, int MODE>
constexpr bool kK32 = sizeof(KT) == 2 && MODE == kExact;

template <int D>
struct PageRegs<D, float> {
    f4 k[D / 16];
    f4 v[4][D / 64];
};

template <int D>
struct PageRegs<D, _Float16> {
    h4 k[D / 16];
    h4 v[4][D / 64];
};

template <typename KT>
struct Raw4;
// Pages are read once per step.  The exact-shape page loads (load_page) each
// take a whole 128-byte line or a contiguous half of one, and carry the
// non-temporal hint (cache policy bit nt = 2): a Qwen2.5-7B-shape decode step
// (64 rows, fp32 pages, 329 MB read cache-cold) measured 63.3-63.9 us with it
// against 67.6-68.2 us without.  On 8-byte fp16 K pieces (a quarter line per
// load) the same hint made fp16 decode steps about 18% slower, which is why
// fp16 K rows are read in the K = 32 layout (16-byte pieces, half a line):
// with it, a Llama-3-8B-shape step (1.7 GB) went from 287.6 to 271.1 us.
constexpr int kStreamLoad = 2;

template <>
struct Raw4<float> {
    typedef f4 T;
    template <int AUX = 0>
    __device__ static f4 load(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4, 0, AUX));
    }
};
template <>
struct Raw4<_Float16> {
    typedef h4 T;
    template <int AUX = 0>
    __device__ static h4 load(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, off * 2, 0, AUX));
    }
};

// Two consecutive elements at element offset `off`.
template <typename KT>
struct Raw2;
template <>
struct Raw2<float> {
    typedef f2 T;
    __device__ static f2 load(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(r, off * 4, 0, 0));
    }
};
template <>
struct Raw2<_Float16> {
    typedef h2 T;
    __device__ static h2 load(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(h2, __builtin_amdgcn_raw_buffer_load_b32(r, off * 2, 0, 0));
    }
};

// One element at element offset `off`.
template <typename KT>
struct Raw1;
template <>
struct Raw1<float> {
    __device__ static float load(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off * 4, 0, 0));
    }
};
template <>
struct Raw1<_Float16> {
    __device__ static _Float16 load(__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, off * 2, 0, 0));
    }
};

// Four elements of a row at dims dim .. dim+3 (element offset `row + dim`),
// zero past `width`, as one piece (kVec4), two (kVec2) or four (kVec1).
template <typename KT, int MODE>
__device__ __forceinline__ typename Raw4<KT>::T load4(__amdgpu_buffer_rsrc_t r, int row, int dim, int width) {
    if constexpr (MODE == kVec1) {
        typename Raw4<KT>::T x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = Raw1<KT>::load(r, dim + i < width ? row + dim + i : kOutOfRange);
        return x;
    } else if constexpr (MODE == kVec2) {
        const auto lo = Raw2<KT>::load(r, dim < width ? row + dim : kOutOfRange);
        const auto hi = Raw2<KT>::load(r, dim + 2 < width ? row + dim + 2 : kOutOfRange);
        return typename Raw4<KT>::T{lo[0], lo[1], hi[0], hi[1]};
    } else {
        return Raw4<KT>::load(r, dim < width ? row + dim : kOutOfRange);
    }
}

template <int D, typename KT, int MODE>
__device__ __forceinline__ void load_page(PageRegs<D, KT>& pr, const KT* kpage, const KT* vpage, int ntok, int n,
                                          int g, const Geo<D, MODE>& geo) {
    if constexpr (MODE != kExact) {
        // Rows are head_dim (v_head_dim) elements apart; a row past ntok, or
        // dims past the width, read as zero.
        const __amdgpu_buffer_rsrc_t rk = page_rsrc(kpage, ntok * geo.d * (int)sizeof(KT));
        const __amdgpu_buffer_rsrc_t rv = page_rsrc(vpage, ntok * geo.dv * (int)sizeof(KT));
#pragma unroll
        for (int j = 0; j < D / 16; ++j) pr.k[j] = load4<KT, MODE>(rk, n * geo.d, 16 * j + 4 * g, geo.d);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int c = 0; c < D / 64; ++c)
                pr.v[kk][c] = load4<KT, MODE>(rv, (4 * g + kk) * geo.dv, 64 * c + 4 * n, geo.dv);
        return;
    }
    const int bytes = ntok * D * (int)sizeof(KT);
    const __amdgpu_buffer_rsrc_t rk = page_rsrc(kpage, bytes);
    const __amdgpu_buffer_rsrc_t rv = page_rsrc(vpage, bytes);
    // The lane's K and V offsets are formed here at every call (the empty asm
    // keeps them from being hoisted out of the page loop), so each load takes
    // its constant part in the instruction's immediate offset.  Hoisted, the
    // sixteen offsets would each hold a register across the loop.
    int kl = n * D + (sizeof(KT) == 2 ? 8 : 4) * g;  // fp16: the K = 32 layout
    int vl = 4 * g * D + 4 * n;
    asm volatile("" : "+v"(kl), "+v"(vl));
    if constexpr (sizeof(KT) == 2) {
        // K = 32 layout: 16 bytes at 32 j + 8 g, half a line of the row.
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
            const h8 x = __builtin_bit_cast(
                h8, __builtin_amdgcn_raw_buffer_load_b128(rk, (kl + 32 * j) * 2, 0, kStreamLoad));
            pr.k[2 * j] = __builtin_shufflevector(x, x, 0, 1, 2, 3);
            pr.k[2 * j + 1] = __builtin_shufflevector(x, x, 4, 5, 6, 7);
        }
    } else {
#pragma unroll
        for (int j = 0; j < D / 16; ++j) pr.k[j] = Raw4<KT>::template load<kStreamLoad>(rk, kl + 16 * j);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int c = 0; c < D / 64; ++c)
            pr.v[kk][c] = Raw4<KT>::template load<kStreamLoad>(rv, vl + kk * D + 64 * c);  // whole lines
}

// Step metadata (unit records, bin offsets, block table) is read-only while
// the kernel runs.  Reading it through the constant address space lets the
// compiler use scalar loads even though the epilogue stores inside the bin
// loop: a vector load there would be followed by a full vmcnt(0) wait that
// also drains the page loads in flight.
typedef __attribute__((address_space(4))) const int32_t const_i32;

__device__ __forceinline__ int ld_meta(const int32_t* p) { return *(const_i32*)p; }

// Four elements of a row at dims dim .. dim + 3 through a plain pointer: zero
// past `width` and for a row that is not valid, in the pieces of MODE.
template <typename KT, int MODE>
__device__ __forceinline__ typename Raw4<KT>::T row4(const KT* row, int dim, int width, bool valid) {
    typedef typename Raw4<KT>::T T4;
    T4 x = {};
    if constexpr (MODE == kVec4) {
        if (valid && dim < width) x = *reinterpret_cast<const T4*>(row + dim);
    } else if constexpr (MODE == kVec2) {
        typedef KT T2 __attribute__((ext_vector_type(2)));
        if (valid && dim < width) {
            const T2 lo = *reinterpret_cast<const T2*>(row + dim);
            x[0] = lo[0];
            x[1] = lo[1];
        }
        if (valid && dim + 2 < width) {
            const T2 hi = *reinterpret_cast<const T2*>(row + dim + 2);
            x[2] = hi[0];
            x[3] = hi[1];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (valid && dim + i < width) x[i] = row[dim + i];
    }
    return x;
}

// Tile t of a row made of m > 1 pages (bt: the row's block ids; blk: page
// t m's block, already read): rows j bs .. j bs + bs - 1 come from block
// bt[t m + j], read only for pages that hold rows below ntok.  Each lane reads
// its K row and its four V rows through plain pointers, so every lane of a
// load fetches (a page tile of 8 tokens leaves half of them idle).
template <int D, typename KT, int MODE>
__device__ __forceinline__ void load_small_pages(PageRegs<D, KT>& pr, const DecodeArgs& a, const KT* kbase,
                                                 const KT* vbase, const int32_t* bt, int t, int64_t blk, int ntok,
                                                 int n, int g, const Geo<D, MODE>& geo) {
    const int bs = geo.bs;
    const int sh = bs == 8 ? 3 : 2;  // m > 1 only for 4- and 8-token pages
    const int* tb = bt + t * geo.m;
    const int b1 = bs < ntok ? ld_meta(tb + 1) : 0;
    const int b2 = geo.m > 2 && 2 * bs < ntok ? ld_meta(tb + 2) : 0;
    const int b3 = geo.m > 3 && 3 * bs < ntok ? ld_meta(tb + 3) : 0;
    auto block_of = [&](int j) -> int64_t { return j == 0 ? blk : j == 1 ? b1 : j == 2 ? b2 : b3; };
    {
        const int j = n >> sh;
        const KT* krow = kbase + block_of(j) * a.block_stride + (int64_t)(n - (j << sh)) * geo.d;
#pragma unroll
        for (int jj = 0; jj < D / 16; ++jj) pr.k[jj] = row4<KT, MODE>(krow, 16 * jj + 4 * g, geo.d, n < ntok);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int rv = 4 * g + kk;
        const int j = rv >> sh;
        const KT* vrow = vbase + block_of(j) * a.v_block_stride + (int64_t)(rv - (j << sh)) * geo.dv;
#pragma unroll
        for (int c = 0; c < D / 64; ++c) pr.v[kk][c] = row4<KT, MODE>(vrow, 64 * c + 4 * n, geo.dv, rv < ntok);
    }
}

// Tile t of a unit's row: one page (block blk) read by load_page, or several
// small pages (load_small_pages).
template <int D, typename KT, int MODE>
__device__ __forceinline__ void load_tile(PageRegs<D, KT>& pr, const DecodeArgs& a, const KT* kbase, const KT* vbase,
                                          const int32_t* bt, int t, int64_t blk, int ntok, int n, int g,
                                          const Geo<D, MODE>& geo) {
    if constexpr (MODE != kExact) {
        if (geo.m > 1) {
            load_small_pages<D, KT, MODE>(pr, a, kbase, vbase, bt, t, blk, ntok, n, g, geo);
            return;
        }
    }
    load_page<D, KT, MODE>(pr, kbase + blk * a.block_stride, vbase + blk * a.v_block_stride, ntok, n, g, geo);
}

// Q^T operand of a unit, q[j] = Q[head n][16j + 4g .. +3], and `sc`, the
// factor that turns the lane's S column (head n) into log2 units.  The
// attention scale multiplies the finished dot, as in the reference
// (PagedAttentionKernel.cs:65).  Heads n >= G of the 16-wide tile read the
// group's head 0: their S, P and O columns stay finite and are never stored.
//  - fp32 pages: q in fp32, sc = scale * log2 e.
//  - fp16 pages: the matrix cores take fp16 operands.  K is exact in fp16;
//    Q is cut into q_hi + q_lo fp16 halves after scaling head n by 2^s_n so
//    that its largest |element| lies in [2^12, 2^13): q_hi + q_lo then
//    carries ~22 significant bits of every element, and sc folds 2^-s_n back.
// The raw fp32 rows are loaded into QRaw ahead of the unit (load_q, no
// arithmetic on the loaded values, so nothing waits for them there) and
// turned into the operand when the unit starts (prepare_q).
template <int D>
struct QRaw {
    f4 q[D / 16];
};

template <int D, typename KT>
struct QRegs;

template <int D>
struct QRegs<D, float> {
    f4 q[D / 16];
    float sc;
};

template <int D>
struct QRegs<D, _Float16> {
    h4 hi[D / 16];
    h4 lo[D / 16];
    float sc;
};

// Q row of head `h` (the tile's head n, or its first head for padding
// lanes); dims past head_dim are zero.
template <int D, typename KT, int MODE>
__device__ __forceinline__ void load_q(QRaw<D>& qr, const DecodeArgs& a, int qi, int h, int g, const Geo<D, MODE>& geo) {
    const float* qrow = a.q + ((int64_t)qi * a.n_heads + h) * geo.d;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
        // q[j] holds dims 16 j + 4 g .. + 3, or for the K = 32 step dims
        // 32 (j / 2) + 8 g + 4 (j % 2) .. + 3 (q[2j], q[2j + 1]: one operand).
        const int dim = kK32<KT, MODE> ? 32 * (j >> 1) + 8 * g + 4 * (j & 1) : 16 * j + 4 * g;
        if constexpr (MODE == kExact) {
            qr.q[j] = *reinterpret_cast<const f4*>(qrow + dim);
        } else if constexpr (MODE == kVec4) {
            qr.q[j] = dim < geo.d ? *reinterpret_cast<const f4*>(qrow + dim) : f4{0.f, 0.f, 0.f, 0.f};
        } else if constexpr (MODE == kVec1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) qr.q[j][i] = dim + i < geo.d ? qrow[dim + i] : 0.f;
        } else {
            const f2 lo = dim < geo.d ? *reinterpret_cast<const f2*>(qrow + dim) : f2{0.f, 0.f};
            const f2 hi = dim + 2 < geo.d ? *reinterpret_cast<const f2*>(qrow + dim + 2) : f2{0.f, 0.f};
            qr.q[j] = f4{lo[0], lo[1], hi[0], hi[1]};
        }
    }
}

template <int D>
__device__ __forceinline__ void prepare_q(QRegs<D, float>& qr, const QRaw<D>& raw, const DecodeArgs& a) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) qr.q[j] = raw.q[j];
    qr.sc = a.scale_log2;
}

template <int D>
__device__ __forceinline__ void prepare_q(QRegs<D, _Float16>& qr, const QRaw<D>& raw, const DecodeArgs& a) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < D / 16; ++j)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(raw.q[j][0]), fabsf(raw.q[j][1])),
                             fmaxf(fabsf(raw.q[j][2]), fabsf(raw.q[j][3]))));
    mx = fmaxf(mx, __shfl_xor(mx, 16));  // head n's elements live in lanes n + 16g
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    int ex = 0;
    if (mx > 0.f) (void)frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
    // Scaled max in [2^12, 2^13); clamped so that 2^sh and 2^-sh stay normal
    // floats.  The floor -115 keeps every finite head inside the fp16 range.
    const int sh = mx > 0.f ? min(100, max(-115, 13 - ex)) : 0;
    const float up = ldexpf(1.0f, sh);
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
        const f4 x = raw.q[j] * up;
        const h4 hi = __builtin_convertvector(x, h4);
        qr.hi[j] = hi;
        qr.lo[j] = __builtin_convertvector(x - __builtin_convertvector(hi, f4), h4);
    }
    qr.sc = ldexpf(a.scale_log2, -sh);
}

template <int D>
struct WaveState {
    f4 o[D / 16];  // O[head 4g + r][64c + 4n + i] for block b = 4c + i
    float m;       // running max (log2 units) of head n
    float l;       // partial sum of head n over this lane's tokens
};

// S^T = K . Q^T for one page; returns the lane's S[head n][token 4g + r] in log2 units.
template <int D, bool K32>
__device__ __forceinline__ f4 page_scores(const PageRegs<D, float>& pr, const QRegs<D, float>& qr) {
    // 32 (d = 128) or 16 (d = 64) rank-4 steps, two accumulation chains.
    f4 s0 = {0.f, 0.f, 0.f, 0.f};
    f4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (j & 1)
                s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(pr.k[j][i], qr.q[j][i], s1, 0, 0, 0);
            else
                s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(pr.k[j][i], qr.q[j][i], s0, 0, 0, 0);
        }
    }
    return (s0 + s1) * qr.sc;
}

template <int D, bool K32>
__device__ __forceinline__ f4 page_scores(const PageRegs<D, _Float16>& pr, const QRegs<D, _Float16>& qr) {
    // K . (q_hi + q_lo), fp32 accumulation: one rank-32 step per 32 dims and
    // half (K32), else one rank-16 step per 16 dims and half.
    f4 s0 = {0.f, 0.f, 0.f, 0.f};
    f4 s1 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (K32) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
            const h8 k = __builtin_shufflevector(pr.k[2 * j], pr.k[2 * j + 1], 0, 1, 2, 3, 4, 5, 6, 7);
            const h8 qh = __builtin_shufflevector(qr.hi[2 * j], qr.hi[2 * j + 1], 0, 1, 2, 3, 4, 5, 6, 7);
            const h8 ql = __builtin_shufflevector(qr.lo[2 * j], qr.lo[2 * j + 1], 0, 1, 2, 3, 4, 5, 6, 7);
            s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k, qh, s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k, ql, s1, 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int j = 0; j < D / 16; ++j) {
            s0 = __builtin_amdgcn_mfma_f32_16x16x16f16(pr.k[j], qr.hi[j], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x16f16(pr.k[j], qr.lo[j], s1, 0, 0, 0);
        }
    }
    return (s0 + s1) * qr.sc;
}

// O += P . V for one page; p = the lane's P[head n][token 4g + r].
template <int D>
__device__ __forceinline__ void page_pv(WaveState<D>& st, const PageRegs<D, float>& pr, const f4& p) {
    // 4 token steps x D/16 output blocks.
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int c = 0; c < D / 64; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st.o[4 * c + i] =
                    __builtin_amdgcn_mfma_f32_16x16x4f32(p[kk], pr.v[kk][c][i], st.o[4 * c + i], 0, 0, 0);
}

template <int D>
__device__ __forceinline__ void page_pv(WaveState<D>& st, const PageRegs<D, _Float16>& pr, const f4& p) {
    // P = p_hi + p_lo in fp16 (P is in [0, 1]); V is exact in fp16.  Output
    // block 4c + i takes B[token 4g + kk][col] = V[4g + kk][64c + 4n + i],
    // i.e. element i of the lane's four V pieces.
    // P arrives times 2^12 (compute_page), so p_lo of a typical probability is a
    // normal fp16 number: the matrix cores flush fp16 subnormals.
    const h4 ph = __builtin_convertvector(p, h4);
    const h4 pl = __builtin_convertvector(p - __builtin_convertvector(ph, f4), h4);
#pragma unroll
    for (int c = 0; c < D / 64; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const h4 b = {pr.v[0][c][i], pr.v[1][c][i], pr.v[2][c][i], pr.v[3][c][i]};
            st.o[4 * c + i] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, b, st.o[4 * c + i], 0, 0, 0);
            st.o[4 * c + i] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, b, st.o[4 * c + i], 0, 0, 0);
        }
}

template <int D, typename KT, int MODE>
__device__ __forceinline__ void compute_page(WaveState<D>& st, const PageRegs<D, KT>& pr, const QRegs<D, KT>& qr,
                                             int ntok, int g) {
#pragma clang fp contract(off)  // the max and the exponents see the same rounded scores
    f4 s = page_scores<D, kK32<KT, MODE>>(pr, qr);
    if (ntok < kTileTokens) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r >= ntok) s[r] = -INFINITY;
    }
    float mp = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mp = fmaxf(mp, __shfl_xor(mp, 16));
    mp = fmaxf(mp, __shfl_xor(mp, 32));
    const float mn = fmaxf(st.m, mp);
    const float alpha = fast_exp2(st.m - mn);  // 0 on the first page (m = -inf)
    st.m = mn;
    f4 p;
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(s[r] - mn);
    // fp16 pages feed P to the matrix cores times 2^12 (page_pv); O and l then
    // carry the same factor, which cancels in O / l.
    const float pscale = sizeof(KT) == 2 ? 4096.0f : 1.0f;
    p *= pscale;
    st.l = st.l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    // O rows are heads 4g + r; their alphas live in lanes 4g + r.
    if (__any(alpha != 1.0f)) {
        const int lane = threadIdx.x & 63;
        const int src = 4 * (lane >> 4);
        f4 ar;
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, src + r);
#pragma unroll
        for (int b = 0; b < D / 16; ++b) st.o[b] *= ar;
    }
    page_pv<D>(st, pr, p);
}

// The scalar fields of unit `ui`; the block ids are read separately (first_block).
__device__ __forceinline__ DecodeUnit read_unit(const DecodeArgs& a, int ui) {
    const int32_t* src = reinterpret_cast<const int32_t*>(a.units + ui);
    DecodeUnit u;
    u.qi = ld_meta(src + 0);
    u.bt_base = ld_meta(src + 1);
    u.page_begin = ld_meta(src + 2);
    u.page_end = ld_meta(src + 3);
    u.ctx = ld_meta(src + 4);
    u.kvh = ld_meta(src + 5);
    u.slot = ld_meta(src + 6);
    u.split_info = ld_meta(src + 7);
    return u;
}

// The block id of this wave's first page of unit `ui` (page_begin + wave),
// which travels in the unit record so the first load needs no table lookup.
// It is read from the record in memory with wave-uniform indices: a local
// copy indexed by `wave` would live in per-lane memory and turn the page
// address divergent.
__device__ __forceinline__ int first_block(const DecodeArgs& a, int ui, int wave) {
    return ld_meta(reinterpret_cast<const int32_t*>(a.units + ui) + 8 + wave);
}

// The same for the wave's second page (page_begin + wave + kDecodeWaves).
__device__ __forceinline__ int second_block(const DecodeArgs& a, int ui, int wave) {
    return ld_meta(reinterpret_cast<const int32_t*>(a.units + ui) + 12 + wave);
}

template <int D, typename KT, int MODE>
__device__ __forceinline__ void load_first_page(PageRegs<D, KT>& pr, const DecodeArgs& a, const DecodeUnit& u, int blk,
                                                int wave, int n, int g, const Geo<D, MODE>& geo) {
    const int p = u.page_begin + wave;
    if (p < u.page_end) {
        const KT* kbase = static_cast<const KT*>(a.k_pool) + a.layer_offset + (int64_t)u.kvh * a.head_stride;
        const KT* vbase = static_cast<const KT*>(a.v_pool) + a.v_layer_offset + (int64_t)u.kvh * a.v_head_stride;
        load_tile<D, KT, MODE>(pr, a, kbase, vbase, a.bt_ids + u.bt_base, p, blk, min(geo.tt, u.ctx - p * geo.tt), n,
                               g, geo);
    }
}

// One workgroup per (bin, tile of heads): for bin bx (blockIdx.x of the
// decode kernel) unit bx, then units [bin_rest[bx], bin_rest[bx + 1]), back to
// back, for the tile `by` (blockIdx.y) of each unit's GQA group.  Before a unit's epilogue (wave merge, output or
// partial) the next unit's Q and first pages are already requested, so the
// CU's load stream keeps going across unit boundaries.
//
// A split piece's partial is published without waiting for it.  The split
// counter protocol then runs at points where waiting is free: at the end of
// the next unit's page loop every wave has no load outstanding, so its wait
// for the partial's stores costs nothing; after the epilogue's barrier (all
// waves' stores complete) lane 0 bumps the pair's counter, behind the next
// unit's prefetch.  The counter's answer is read at the end of the following
// page loop, again with nothing else in flight, and the last split of a pair
// merges it in that unit's epilogue.  A workgroup's last one or two pieces settle after its
// final unit.
template <int D, typename KT, int MODE>
__device__ __forceinline__ void decode_bins_body(const DecodeArgs& a, EpilogueLds<D, kMaxGroupMfma>& sh, int bx,
                                                 int by) {

    const Geo<D, MODE> geo(a);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;
    const int g = lane >> 4;
    const int first = bx;

    // This workgroup's tile of the group: heads [hoff, hoff + G).
    Tile t;
    t.hoff = kDecodeTileHeads * by;
    t.G = min(kDecodeTileHeads, a.group - t.hoff);
    t.gs = a.slot_heads;
    t.dv = geo.dv;
    {
        const int64_t tile = by;
        t.part_o = a.part_o ? a.part_o + tile * a.num_slots * a.slot_heads * geo.dv : nullptr;
        t.part_ml = a.part_ml ? a.part_ml + tile * a.num_slots * a.slot_heads * 2 : nullptr;
        t.counters = a.counters ? a.counters + tile * a.total_q * a.n_kv : nullptr;
    }
    const int G = t.G;
    // Heads n >= G of the 16-wide tile read the tile's first head: their S, P
    // and O columns stay finite and are never stored.
    const int hq = t.hoff + (n < G ? n : 0);

    QRaw<D> qraw;
    PageRegs<D, KT> ra, rb;
    {
        const DecodeUnit u0 = read_unit(a, first);
        const int blk0 = first_block(a, first, wave);
        load_q<D, KT, MODE>(qraw, a, u0.qi, u0.kvh * a.group + hq, g, geo);
        load_first_page<D, KT, MODE>(ra, a, u0, blk0, wave, n, g, geo);
    }
    const int rb0 = ld_meta(a.bin_rest + first);
    const int re = ld_meta(a.bin_rest + first + 1);
    bool rb_ready = false;  // rb already holds page p + kDecodeWaves (prefetched across a boundary)

    int pub = -1;      // split unit whose partial is stored but not yet counted
    int cnt = -1;      // split unit whose count is in flight (answer in `counted`, lane 0 of wave 0)
    int counted = 0;

    // The unit record is re-read from memory in every iteration (wave-uniform
    // address), never carried across iterations, so every field stays scalar.
    for (int k = rb0 - 1; k < re; ++k) {
        const int ui = k < rb0 ? first : k;
        const DecodeUnit u = read_unit(a, ui);
        QRegs<D, KT> q;
        prepare_q<D>(q, qraw, a);
        const bool has_next = k + 1 < re;
        // The next record and its first two page ids are fetched now; their
        // latency hides behind this unit.
        const DecodeUnit un = read_unit(a, has_next ? k + 1 : ui);
        const int blkn = first_block(a, has_next ? k + 1 : ui, wave);
        const int pn2 = un.page_begin + wave + kDecodeWaves;  // the next unit's second page of this wave
        const bool has_n2 = has_next && pn2 < un.page_end;
        const int blkn2 = second_block(a, has_next ? k + 1 : ui, wave);

        WaveState<D> st;
#pragma unroll
        for (int b = 0; b < D / 16; ++b) st.o[b] = f4{0.f, 0.f, 0.f, 0.f};
        st.m = -INFINITY;
        st.l = 0.f;

        const KT* kbase = static_cast<const KT*>(a.k_pool) + a.layer_offset + (int64_t)u.kvh * a.head_stride;
        const KT* vbase = static_cast<const KT*>(a.v_pool) + a.v_layer_offset + (int64_t)u.kvh * a.v_head_stride;
        const int32_t* bt = a.bt_ids + u.bt_base;

        // Two page buffers in flight: load page p + kDecodeWaves while computing page p.
        int p = u.page_begin + wave;
        while (p < u.page_end) {
            const int pn = p + kDecodeWaves;
            if (pn < u.page_end && !rb_ready) {
                const int64_t blk = ld_meta(bt + pn * geo.m);
                load_tile<D, KT, MODE>(rb, a, kbase, vbase, bt, pn, blk, min(geo.tt, u.ctx - pn * geo.tt), n, g, geo);
            }
            rb_ready = false;
            compute_page<D, KT, MODE>(st, ra, q, min(geo.tt, u.ctx - p * geo.tt), g);
            if (pn >= u.page_end) break;
            const int pnn = pn + kDecodeWaves;
            if (pnn < u.page_end) {
                const int64_t blk = ld_meta(bt + pnn * geo.m);
                load_tile<D, KT, MODE>(ra, a, kbase, vbase, bt, pnn, blk, min(geo.tt, u.ctx - pnn * geo.tt), n, g,
                                       geo);
            }
            compute_page<D, KT, MODE>(st, rb, q, min(geo.tt, u.ctx - pn * geo.tt), g);
            p = pnn;
        }

        // No page load is outstanding here, so these waits are free: the
        // count in flight comes back (read by every lane, so that on every
        // path it is done here), and this wave's stores of `pub` complete.
        const int prev = __builtin_amdgcn_readfirstlane(counted);
        if (pub >= 0) wait_vm_complete();

        // Both page buffers and q are free now: request the next unit's Q and
        // first two pages of this wave, so the epilogue runs with two pages
        // per wave in flight.
        rb_ready = false;
        if (has_next) {
            load_q<D, KT, MODE>(qraw, a, un.qi, un.kvh * a.group + hq, g, geo);
            load_first_page<D, KT, MODE>(ra, a, un, blkn, wave, n, g, geo);
            if (has_n2) {
                const KT* nkbase = static_cast<const KT*>(a.k_pool) + a.layer_offset + (int64_t)un.kvh * a.head_stride;
                const KT* nvbase =
                    static_cast<const KT*>(a.v_pool) + a.v_layer_offset + (int64_t)un.kvh * a.v_head_stride;
                load_tile<D, KT, MODE>(rb, a, nkbase, nvbase, a.bt_ids + un.bt_base, pn2, blkn2,
                                       min(geo.tt, un.ctx - pn2 * geo.tt), n, g, geo);
                rb_ready = true;
            }
        }

        // Per-head sums over the four lane groups; m is uniform per head already.
        st.l += __shfl_xor(st.l, 16);
        st.l += __shfl_xor(st.l, 32);
        if (g == 0 && n < G) {
            sh.m[wave][n] = st.m;
            sh.l[wave][n] = st.l;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            if (h < G) {
#pragma unroll
                for (int c = 0; c < D / 64; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) sh.o[wave][h][64 * c + 4 * n + i] = st.o[4 * c + i][r];
            }
        }
        if (cnt >= 0 && tid == 0) sh.last = prev == (read_unit(a, cnt).split_info >> 16) - 1;
        __syncthreads();
        // Every wave has waited for its part of `pub`'s partial: count it.
        // The answer is read at the end of the next page loop.
        if (pub >= 0 && tid == 0) counted = count_split(a, read_unit(a, pub), t);
        const bool merge_cnt = cnt >= 0 && sh.last;
        publish_unit<D, kMaxGroupMfma>(a, u, t, sh);
        if (merge_cnt) merge_pair<D, kMaxGroupMfma, 0>(a, read_unit(a, cnt), t, sh);
        cnt = pub;
        pub = (u.split_info >> 16) > 1 ? ui : -1;
        __syncthreads();  // the epilogue LDS is reused by the next unit
    }

    // Settle the last pieces: `cnt` has a count in flight, `pub` none yet.
    if (cnt >= 0 || pub >= 0) {
        const int prev = __builtin_amdgcn_readfirstlane(counted);
        wait_vm_complete();
        __syncthreads();
        int prev_pub = 0;
        if (pub >= 0 && tid == 0) prev_pub = count_split(a, read_unit(a, pub), t);
        if (tid == 0) {
            sh.last = cnt >= 0 && prev == (read_unit(a, cnt).split_info >> 16) - 1;
            sh.last_pub = pub >= 0 && prev_pub == (read_unit(a, pub).split_info >> 16) - 1;
        }
        __syncthreads();
        if (sh.last) merge_pair<D, kMaxGroupMfma>(a, read_unit(a, cnt), t, sh);
        if (sh.last_pub) merge_pair<D, kMaxGroupMfma>(a, read_unit(a, pub), t, sh);
    }
}

}  // namespace
}  // namespace gsp
