// Matrix-core (MFMA) kernel for chunked-prefill rows of the paged-attention
// step, gfx950.
//
// A prefill row stores its whole chunk first, then query token i attends to
// min(TokenCount, pos + i + 1) tokens (PagedTransformerRunner.cs:425-474,
// PagedAttentionKernel.cs:41).  Its queries share every K/V page of the prefix,
// so the work is a dense causal contraction; one workgroup owns a tile of 16
// consecutive query tokens of one row and one KV head, for up to 8 query heads
// of the GQA group (4 when the group has at most 4; grid.y covers larger
// groups), and walks the row's pages in
// order:
//
//   per pair of pages (32 keys, staged once in LDS and shared by the group's heads):
//     S^T[key][token] = K_page . Q_head^T   (per page: M = keys, N = tokens, K = head dim)
//     O_head[token][e] += P . V_pair          (M = tokens, N = head dim, K = 32 keys)
//
// with fp32 accumulation, on v_mfma_f32_16x16x32_f16 (on gfx950 it does twice
// the work of v_mfma_f32_16x16x16f16 in the same cycles): QK takes 32 head
// dims per step, and PV 32 keys, so pages go in pairs.  Operands enter as
// fp16 pairs x = x_hi + x_lo, each side scaled by a power of two so that its
// largest element lies in [2^12, 2^13) (the pair then carries ~22
// significant bits and nothing overflows or flushes):
//   - Q: per query token (the lane's S column), at load;
//   - fp32 K, V pages: per key row, while the page is staged into LDS;
//     fp16 pages are exact in fp16 and enter as they are (x_lo = 0);
//   - P: times 2^12, so that p_lo stays a normal fp16 number (the matrix
//     cores flush fp16 subnormals; an unscaled p_lo of a typical probability
//     would be one, and P would keep only 11 bits).  P = 2^(s - m) is taken
//     against a max m that lags the running max by at most 2^3 (the O
//     rescale is skipped until a row grows further), so P' < 2^15.
// S = K_hi.Q_hi + K_hi.Q_lo + K_lo.Q_hi (the K_lo.Q_lo term is ~2^-22
// relative), times 2^(e_key + e_token) * scale.  The V scales fold into P:
// the accumulator O is kept in units of 2^(eO - 12), eO the largest V
// exponent seen so far, so P' = P * 2^(e_v(key) - eO + 12) < 2^15, and O is
// rescaled (like the softmax's alpha) when a page raises eO.  Precision bound
// of that fold: a key whose V row is more than ~2^14 smaller than the row's
// largest V row gets a subnormal P' and keeps fewer bits (none beyond ~2^26);
// its absolute error stays below ~2^-25 of the largest |V| element.
//
// Row tile T of the workgroup is query head hc + T over the 16 tokens; wave w
// owns tiles w and w + 4 (or tile w alone, for groups of at most 4).  The MFMA operand layouts are the decode kernel's
// with "head" replaced by "query token" (lane l, n = l % 16, g = l / 16):
//   QK A = K[key n][32j + 8g .. +7], B = Q[token n][32j + 8g .. +7]
//   result: lane holds S[token n][key 4g + r]
//   PV A = P'[token n][the lane's own eight keys: 4g .. 4g+3 of each page of the pair],
//   B = V[the same eight keys][col], col = 64c + 4n + i for output block 4c + i;
//   result: lane holds O[token 4g + r][col].
// The causal limit is per row (token); padding rows past the tile's tokens
// keep finite scores and are never written.  Page pairs are staged through two
// LDS buffers with one barrier per pair; V goes in transposed, so each PV B
// operand is one 16-byte LDS read, and the K and V operands of the next
// matrix step are read while the current one runs.
//
// Two forms for fp32 pages.  Every tile of a row reads the same page pairs, so
// by default (split records) prefill_split_kernel first writes each pair of
// each tiled row and KV head once per step and layer as the finished image of
// an LDS buffer (hi/lo K rows with one K exponent for the pair, transposed
// hi/lo V with per-key exponents, the scales), and the tiles copy records into
// LDS with direct-to-LDS loads: no staging registers, no split arithmetic in
// the tile, and the score products of pair k overlap the softmax of pair
// k - 1 (prefill_tile_body_rec).  Without records (the allocation-free entry
// point, fp16 pages) each tile stages and splits the pages it reads through
// registers, a page at a time (prefill_tile_body).
// The roofline of these rows is the matrix peak.
#include "gsp_decode_body.h"

#include <type_traits>

namespace gsp {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kPScaleLog2 = 12;  // P enters the matrix cores times 2^12 (p_lo stays normal)
static_assert(kPrefillTileTokens == kBlockSize, "the tile's token and key dimensions are both 16");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t prefill_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// Exponent e such that x * 2^-e has its largest |element| `mx` in [2^12, 2^13).
// Clamped to [-100, 115] so that 2^-e and 2^e stay normal floats (inputs below
// 2^-87 then keep their absolute fp16 rounding only); the ceiling keeps every
// finite vector inside the fp16 range.  An all-zero vector
// (such as the slots past a page's valid tokens, which load as 0) gets the
// floor -100, so it never raises the largest V exponent of a page.
constexpr int kPairExpFloor = -100;
constexpr int kPairExpCeil = 115;
__device__ __forceinline__ int pair_exponent(float mx) {
    int ex = 0;
    if (mx > 0.f) (void)frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
    return mx > 0.f ? min(kPairExpCeil, max(kPairExpFloor, ex - 13)) : kPairExpFloor;
}

template <typename F, typename H>
__device__ __forceinline__ void split_pair(const F& x, H& hi, H& lo) {
    hi = __builtin_convertvector(x, H);
    lo = __builtin_convertvector(x - __builtin_convertvector(hi, F), H);
}

__device__ __forceinline__ float max_abs4(const f4& x) {
    return fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
}

template <typename T, int W>
struct VecW {
    typedef T type __attribute__((ext_vector_type(W)));
};

// STREAM: the non-temporal hint for data read once (16-byte loads only; see
// kStreamLoad).
template <typename V, bool STREAM = false>
__device__ __forceinline__ V buffer_load(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (sizeof(V) == 16)
        return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, STREAM ? kStreamLoad : 0));
    else if constexpr (sizeof(V) == 8) return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    else return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Page staging.  K: key row tid / 16 is moved by the 16 lanes of one DPP row;
// lane part = tid % 16 moves the D / 64 four-element chunks at columns
// 64 j + 4 part (each load instruction reads 256 contiguous bytes per row).
// V: lane vpart = tid % 32 moves columns kVW * vpart .. + kVW - 1 of the two
// keys 2 kg and 2 kg + 1, kg = tid / 32, so that it can store each column's
// key pair as one 32-bit word of the transposed V (below).
template <int D>
constexpr int kStageChunks = D / 64;
template <int D>
constexpr int kVW = D / 32;
static_assert(kBlockSize * 16 == kDecodeThreads, "one 16-lane row per key of the page");
static_assert(kBlockSize / 2 * 32 == kDecodeThreads, "one 32-lane half-wave per key pair of the page");

template <int D, typename KT>
struct PfStage {
    typedef KT kvec __attribute__((ext_vector_type(4)));
    typedef typename VecW<KT, kVW<D>>::type vvec;
    kvec k[kStageChunks<D>];
    vvec v[2];  // keys 2 kg and 2 kg + 1
};

// LDS buffers (two), each holding a pair of pages: keys 0..15 of the first
// page, then 16..31 of the second.  K rows are padded by 8 halves (16 bytes).
// V is stored transposed, one row per column, with the keys in the order the
// P.V step consumes them: position 8 q + 4 h + r holds key 4 q + r of page h,
// so lane group g reads its eight keys (4g .. 4g + 3 of each page) as one
// 16-byte word.  A row of fp32 pages holds the 32 hi halves, then the 32 lo
// halves.  Every fourth column row is followed by 8 halves of padding, which
// puts the 16 lanes of one read (columns 4n + i) on distinct banks.
constexpr int kPairKeys = 2 * kBlockSize;

template <bool kSplit>
constexpr int kVtStride = kSplit ? 2 * kPairKeys : kPairKeys;

template <int D, bool kSplit>
constexpr int kVtLen = D * kVtStride<kSplit> + (D / 4) * 8;

template <bool kSplit>
__device__ __forceinline__ constexpr int vt_row(int col) { return col * kVtStride<kSplit> + (col >> 2) * 8; }

template <int D, typename KT>
struct PfLds;

// A buffer of fp32 pages is two halves: the K half (the hi and lo rows) and
// the V half (the transposed V pairs and the scales of both K and V).  Each
// half's arrays sit together, so every offset within a half fits the 16-bit
// immediate of an LDS instruction.  Both halves are 128 (D + 8) bytes, whole
// kilobytes (the span of one wave's 16-byte-per-lane direct-to-LDS load), and
// a buffer is also the layout of a split record (one page pair of one row and
// KV head, written once per step by prefill_split_kernel), so a tile copies a
// record, or either half of one, into LDS with no registers and no arithmetic.
constexpr int kRecordChunk = 64 * 16;
template <int D>
constexpr int kHalfBytes = 2 * kPairKeys * (D + 8) * 2;
template <int D>
constexpr int kRecordBytes = 2 * kHalfBytes<D>;

template <int D>
struct alignas(16) PfKHalf {
    _Float16 kh[kPairKeys * (D + 8)], kl[kPairKeys * (D + 8)];
};

template <int D>
struct alignas(16) PfVHalfBody {
    _Float16 vt[kVtLen<D, true>];
    float ks[kPairKeys];  // 2^e of each key's K pair
    int ev[kPairKeys];    // exponent of each key's V pair
    int evw[2 * kDecodeWaves];          // largest V exponent of each wave's four keys, per page
};

template <int D>
struct alignas(16) PfVHalf : PfVHalfBody<D> {
    unsigned char pad[kHalfBytes<D> - sizeof(PfVHalfBody<D>)];
};

template <int D>
struct alignas(16) PfLdsBuf32 {
    PfKHalf<D> k;
    PfVHalf<D> v;
};
static_assert(sizeof(PfKHalf<128>) == kHalfBytes<128> && sizeof(PfVHalf<128>) == kHalfBytes<128> &&
                  sizeof(PfKHalf<64>) == kHalfBytes<64> && sizeof(PfVHalf<64>) == kHalfBytes<64>,
              "each half is whole kilobytes");
static_assert(kHalfBytes<128> % kRecordChunk == 0 && kHalfBytes<64> % kRecordChunk == 0, "whole chunks");

template <int D>
struct alignas(16) PfLds<D, float> {
    static constexpr int kRow = D + 8;
    PfLdsBuf32<D> b[2];
};

template <int D>
struct alignas(16) PfLdsBuf16 {
    _Float16 k[kPairKeys * (D + 8)];
    _Float16 v[kVtLen<D, false>];
};

template <int D>
struct alignas(16) PfLds<D, _Float16> {
    static constexpr int kRow = D + 8;
    PfLdsBuf16<D> b[2];
};

// Element offset of lane tid's K chunk j in a page (key row tid / 16).
template <int D>
__device__ __forceinline__ int stage_offset(int j) {
    return (threadIdx.x >> 4) * D + 64 * j + 4 * (threadIdx.x & 15);
}

// STREAM: the pages are read once (the split pass), not by every tile of a row.
template <int D, typename KT, bool STREAM = false>
__device__ __forceinline__ void stage_load(PfStage<D, KT>& sr, const KT* kpage, const KT* vpage, int ntok) {
    typedef typename PfStage<D, KT>::kvec kvec;
    typedef typename PfStage<D, KT>::vvec vvec;
    constexpr int kE = (int)sizeof(KT);
    const int bytes = ntok * D * kE;
    const __amdgpu_buffer_rsrc_t rk = prefill_rsrc(kpage, bytes);
    const __amdgpu_buffer_rsrc_t rv = prefill_rsrc(vpage, bytes);
#pragma unroll
    for (int i = 0; i < kStageChunks<D>; ++i) sr.k[i] = buffer_load<kvec, STREAM>(rk, kE * stage_offset<D>(i));
    const int kg = threadIdx.x >> 5;
    const int vpart = threadIdx.x & 31;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) sr.v[kk] = buffer_load<vvec, STREAM>(rv, kE * ((2 * kg + kk) * D + kVW<D> * vpart));
}

// Max of x over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four rows of a wave),
// with the row swaps of gfx950: max of the swapped pair is the max across the
// exchanged rows.
__device__ __forceinline__ float cross_row_max(float x) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// pair_exponent from the bit pattern of mx >= 0: for a normal mx, frexp's
// exponent is the field minus 126; zero and subnormal maxima (field 0) land on
// the floor as above.  Infinite and NaN maxima take the ceiling and stay
// non-finite after scaling.
__device__ __forceinline__ int pair_exponent_bits(uint32_t mb) {
    return min(kPairExpCeil, max(kPairExpFloor, (int)(mb >> 23) - 139));
}

// Largest |x[i]| as a bit pattern: the lane's elements go through
// v_max3_f32 with its free |.| modifiers (written out, because fmaxf of
// loaded values first quiets each input on its own instruction); lanes are
// then combined with integer maxima, since non-negative floats order like
// their bits.
template <typename V>
__device__ __forceinline__ uint32_t max_abs_bits(const V& x) {
    constexpr int kN = (int)(sizeof(V) / sizeof(float));
    static_assert(kN == 2 || kN == 4, "two or four elements");
    float m;
    if constexpr (kN == 4) {
        asm("v_max3_f32 %0, |%1|, |%2|, |%3|" : "=v"(m) : "v"(x[0]), "v"(x[1]), "v"(x[2]));
        asm("v_max_f32_e64 %0, %1, |%2|" : "=v"(m) : "v"(m), "v"(x[3]));
    } else {
        asm("v_max_f32_e64 %0, |%1|, |%2|" : "=v"(m) : "v"(x[0]), "v"(x[1]));
    }
    return __float_as_uint(m);
}

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, kCtrl, 0xF, 0xF, true);
}

// Unsigned max over the 16 lanes of a DPP row (the moves fold into the maxima).
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t x) {
    x = max(x, dpp_u32<0xB1>(x));   // quad_perm [1, 0, 3, 2]
    x = max(x, dpp_u32<0x4E>(x));   // quad_perm [2, 3, 0, 1]
    x = max(x, dpp_u32<0x124>(x));  // row_ror:4
    return max(x, dpp_u32<0x128>(x));  // row_ror:8
}

// Unsigned max over lanes l and l ^ 16.
__device__ __forceinline__ uint32_t swap16_max_u32(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return max(r[0], r[1]);
}

// Signed max over lanes l and l ^ 32.
__device__ __forceinline__ int swap32_max_i32(int x) {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
    return max((int)r[0], (int)r[1]);
}

// K rows take one exponent per key (PAIR_K false) or ek_pair for the whole
// page pair (split records: the scores then need one factor per tile).
template <int D, bool PAIR_K = false>
__device__ __forceinline__ void stage_store(const PfStage<D, float>& sr, PfLdsBuf32<D>& b, int slot, int ek_pair = 0) {
    constexpr int kRow = PfLds<D, float>::kRow;
    constexpr int W = kVW<D>;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const int key = threadIdx.x >> 4;
    const int part = threadIdx.x & 15;
    int ek = ek_pair;
    if constexpr (!PAIR_K) {
        uint32_t mk = 0;
#pragma unroll
        for (int i = 0; i < kStageChunks<D>; ++i) mk = max(mk, max_abs_bits(sr.k[i]));
        ek = pair_exponent_bits(row16_max_u32(mk));
    }
    const float dk = ldexpf(1.0f, -ek);
#pragma unroll
    for (int i = 0; i < kStageChunks<D>; ++i) {
        const int at = (slot * kBlockSize + key) * kRow + 64 * i + 4 * part;
        h4 hi, lo;
        split_pair(sr.k[i] * dk, hi, lo);
        *reinterpret_cast<h4*>(&b.k.kh[at]) = hi;
        *reinterpret_cast<h4*>(&b.k.kl[at]) = lo;
    }
    if (part == 0) b.v.ks[slot * kBlockSize + key] = ldexpf(1.0f, ek);

    // V, transposed: each of the lane's columns takes its key pair as one
    // word of hi halves and one of lo halves.
    const int kg = threadIdx.x >> 5;
    const int vpart = threadIdx.x & 31;
    int ev[2];
    float dv[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        ev[kk] = pair_exponent_bits(swap16_max_u32(row16_max_u32(max_abs_bits(sr.v[kk]))));
        dv[kk] = ldexpf(1.0f, -ev[kk]);
    }
    const int pos = 8 * (kg >> 1) + 4 * slot + 2 * (kg & 1);  // keys 2 kg, 2 kg + 1 of page `slot`
#pragma unroll
    for (int c = 0; c < W; ++c) {
        const int at = vt_row<true>(W * vpart + c) + pos;
        h2 hi, lo;
        split_pair(f2{sr.v[0][c] * dv[0], sr.v[1][c] * dv[1]}, hi, lo);
        *reinterpret_cast<h2*>(&b.v.vt[at]) = hi;
        *reinterpret_cast<h2*>(&b.v.vt[at + kPairKeys]) = lo;
    }
    if (vpart == 0) {
        b.v.ev[slot * kBlockSize + 2 * kg] = ev[0];
        b.v.ev[slot * kBlockSize + 2 * kg + 1] = ev[1];
    }
    // The page's largest V exponent: this wave's four keys (two per half-wave),
    // then one slot per wave.
    const int evw = swap32_max_i32(max(ev[0], ev[1]));
    if ((threadIdx.x & 63) == 0) b.v.evw[slot * kDecodeWaves + (threadIdx.x >> 6)] = evw;
}

template <int D>
__device__ __forceinline__ void stage_store(const PfStage<D, _Float16>& sr, PfLdsBuf16<D>& b, int slot) {
    constexpr int kRow = PfLds<D, _Float16>::kRow;
    constexpr int W = kVW<D>;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const int key = threadIdx.x >> 4;
    const int part = threadIdx.x & 15;
#pragma unroll
    for (int i = 0; i < kStageChunks<D>; ++i) {
        const int at = (slot * kBlockSize + key) * kRow + 64 * i + 4 * part;
        *reinterpret_cast<h4*>(&b.k[at]) = sr.k[i];
    }
    const int kg = threadIdx.x >> 5;
    const int vpart = threadIdx.x & 31;
    const int pos = 8 * (kg >> 1) + 4 * slot + 2 * (kg & 1);
#pragma unroll
    for (int c = 0; c < W; ++c)
        *reinterpret_cast<h2*>(&b.v[vt_row<false>(W * vpart + c) + pos]) = h2{sr.v[0][c], sr.v[1][c]};
}

// Split records of fp32 pages.  Every tile of a row walks the row's pages from
// page 0 in the same pairs, so the hi/lo split of pair i (for one KV head) is
// the same for all of them: prefill_split_kernel writes it once per step as
// the image of one LDS buffer (K half, then V half), and a tile copies the
// halves it needs into LDS with direct-to-LDS loads.  The record of a row's
// pair covers the row's tokens up to min(TokenCount, pos + q_len); keys of it
// past a tile's own limit are masked like any other.

// 16 bytes per lane from r at soffset + voffset into LDS at lds + 16 * lane
// (lds and soffset uniform over the wave).
__device__ __forceinline__ void lds_load16s(__amdgpu_buffer_rsrc_t r, void* lds, int voffset, int soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0,
                                             0);
}

// One half (kHalfBytes) of the record r (a resource over that one record) from
// byte `off` into `dst`: lane l of wave w moves bytes 1024 (4 c + w) + 16 l of
// the half for c = 0, 1, ...; each wave's kilobyte lands contiguously at the
// same offset of dst.  The lane's part of the offset is the same for every
// chunk; the rest is uniform and goes in the scalar offset.
template <int D>
__device__ __forceinline__ void half_load(void* dst, __amdgpu_buffer_rsrc_t r, int off) {
    constexpr int kChunks = kHalfBytes<D> / kRecordChunk;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane_off = 16 * (threadIdx.x & 63);
    unsigned char* base = static_cast<unsigned char*>(dst);
#pragma unroll
    for (int c0 = 0; c0 < kChunks; c0 += kDecodeWaves) {
        const int c = c0 + w;
        if (c0 + kDecodeWaves <= kChunks || c < kChunks)  // only the last round may be partial
            lds_load16s(r, base + kRecordChunk * c, lane_off, off + kRecordChunk * c);
    }
}

// The direct-to-LDS loads of this wave have landed (the barrier after it
// publishes them to the other waves).
__device__ __forceinline__ void record_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// One workgroup per (page pair, row and KV head): stages the pair exactly as
// a tile would (stage_load, stage_store) and writes the buffer out as record
// item.rec0 + pair.  Pairs past the row's pages exit at once.
template <int D>
__global__ __launch_bounds__(kDecodeThreads) void prefill_split_kernel(PrefillSplitArgs a) {
    __shared__ PfLdsBuf32<D> sh;
    const PrefillSplitItem it = a.items[blockIdx.y];
    const int pages = (it.ctx_last + kBlockSize - 1) / kBlockSize;
    const int pair = blockIdx.x;
    if (2 * pair >= pages) return;
    const float* kbase = static_cast<const float*>(a.k_pool) + a.layer_offset + (int64_t)it.kvh * a.head_stride;
    const float* vbase = static_cast<const float*>(a.v_pool) + a.layer_offset + (int64_t)it.kvh * a.head_stride;
    const int32_t* bt = a.bt_ids + it.bt_base;
    PfStage<D, float> sr[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int pg = 2 * pair + h;
        const bool have = pg < pages;
        const int64_t blk = have ? bt[pg] : 0;
        stage_load<D, float, true>(sr[h], kbase + blk * a.block_stride, vbase + blk * a.block_stride,
                      have ? min(kBlockSize, it.ctx_last - pg * kBlockSize) : 0);
    }
    // One K exponent for the pair: its largest |K| over both pages (wave
    // maxima, then the four waves through LDS).
    __shared__ uint32_t wave_max[kDecodeWaves];
    uint32_t mk = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < kStageChunks<D>; ++i) mk = max(mk, max_abs_bits(sr[h].k[i]));
    mk = (uint32_t)swap32_max_i32((int)swap16_max_u32(row16_max_u32(mk)));  // bits of |x| < 2^31
    if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = mk;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) mk = max(mk, wave_max[w]);
    const int ek = pair_exponent_bits(mk);
    stage_store<D, true>(sr[0], sh, 0, ek);
    stage_store<D, true>(sr[1], sh, 1, ek);
    __syncthreads();
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const u4* src = reinterpret_cast<const u4*>(&sh);
    u4* dst = reinterpret_cast<u4*>(a.records + ((int64_t)it.rec0 + pair) * kRecordBytes<D>);
    for (int i = threadIdx.x; i < kRecordBytes<D> / 16; i += kDecodeThreads) dst[i] = src[i];
}

// Q operands of one tile for the K = 32 matrix cores, q[j] = Q[token n][32j + 8g
// .. +7] as a scaled fp16 pair, and the lane's score factor 2^e_token * |scale|
// (log2 units).  Q carries the scale's sign (an exact negation), so the factor
// is positive and the largest score times it is the largest scaled score.
template <int D>
struct TileQ {
    h8 hi[D / 32];
    h8 lo[D / 32];
    float sc;
};

template <int D>
__device__ __forceinline__ void load_tile_q(TileQ<D>& tq, const float* qrow, bool live, int g, float scale) {
    f4 x[D / 16];  // x[2j + h] = Q[token n][32j + 8g + 4h .. +3]
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
        const f4 v = *reinterpret_cast<const f4*>(qrow + 32 * (j >> 1) + 8 * g + 4 * (j & 1));
        x[j] = live ? v : f4{0.f, 0.f, 0.f, 0.f};
        mx = fmaxf(mx, max_abs4(x[j]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));  // token n's elements live in lanes n + 16g
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const int e = pair_exponent(mx);
    const float down = scale < 0.f ? -ldexpf(1.0f, -e) : ldexpf(1.0f, -e);
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
        h4 h0, l0, h1, l1;
        split_pair(x[2 * j] * down, h0, l0);
        split_pair(x[2 * j + 1] * down, h1, l1);
        tq.hi[j] = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
        tq.lo[j] = __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7);
    }
    tq.sc = ldexpf(fabsf(scale), e);
}

// Per-tile softmax state: O (in the wave's units, see eo below), the max m (log2 units) that
// token n's probabilities are taken against, partial sum l of token n over
// this lane's keys.
template <int D>
struct TileState {
    f4 o[D / 16];
    float m;
    float l;
};

// A row's running max may grow this much (log2 units) before O and l are
// rescaled: until then P = 2^(s - m) stays below 2^kLazyLog2, and P' (P times
// at most 2^kPScaleLog2, see below) below 2^15, inside fp16's range.
constexpr float kLazyLog2 = 3.0f;

// Causal mask and online softmax of one page's scores; returns P, and in
// `alpha_rows` the factors that the lane's O rows (tokens 4g + r) must take,
// fetched from the lanes that own those tokens (`rescale` false: all 1).  m
// only moves when some row of the tile has grown by more than kLazyLog2, which
// after the first pages is rare, so most pages skip the O rescale.
template <int D>
__device__ __forceinline__ f4 page_softmax(TileState<D>& st, f4 s, bool diag, int key0, int row_ctx, int g,
                                           f4& alpha_rows, bool& rescale) {
#pragma clang fp contract(off)  // the max and the exponents see the same rounded scores
    if (diag) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (key0 + r >= row_ctx) s[r] = -INFINITY;
    }
    // Token n's page max: its keys live in lanes n + 16g.
    const float mp = cross_row_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
    rescale = __any(mp > st.m + kLazyLog2);  // true on the first page (m = -inf)
    if (rescale) {
        const float mn = fmaxf(st.m, mp);  // finite: page 0 holds key 0 for every row
        const float alpha = fast_exp2(st.m - mn);
        st.m = mn;
        st.l *= alpha;
#pragma unroll
        for (int r = 0; r < 4; ++r) alpha_rows[r] = __shfl(alpha, 4 * g + r);
    }
    f4 p;
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(s[r] - st.m);
    st.l += (p[0] + p[1]) + (p[2] + p[3]);
    return p;
}

// page_softmax over a pair of pages: the lane's eight scores are keys
// key0 + r (first page, s0) and key0 + 16 + r (second page, s1).
template <int D>
__device__ __forceinline__ void pair_softmax(TileState<D>& st, f4& s0, f4& s1, bool diag, int key0, int row_ctx,
                                             int g, f4& alpha_rows, bool& rescale) {
#pragma clang fp contract(off)  // the max and the exponents see the same rounded scores
    if (diag) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (key0 + r >= row_ctx) s0[r] = -INFINITY;
            if (key0 + kBlockSize + r >= row_ctx) s1[r] = -INFINITY;
        }
    }
    const float mp = cross_row_max(fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                         fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3]))));
    rescale = __any(mp > st.m + kLazyLog2);  // true on the first pair (m = -inf)
    if (rescale) {
        const float mn = fmaxf(st.m, mp);  // finite: the first page holds key 0 for every row
        const float alpha = fast_exp2(st.m - mn);
        st.m = mn;
        st.l *= alpha;
#pragma unroll
        for (int r = 0; r < 4; ++r) alpha_rows[r] = __shfl(alpha, 4 * g + r);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s0[r] = fast_exp2(s0[r] - st.m);
        s1[r] = fast_exp2(s1[r] - st.m);
    }
    st.l += ((s0[0] + s0[1]) + (s0[2] + s0[3])) + ((s1[0] + s1[1]) + (s1[2] + s1[3]));
}

// TILES query heads per wave (heads wave + 4 s, s < TILES): 2 for groups above
// 4 heads, else 1.  Every tile of a wave is computed on every page, so the
// hot loop has no branches; a tile past the group (zero Q) is simply not
// stored.  It costs no time: the page barrier waits for the busiest wave.
// This form splits the fp32 pages it reads itself (fp16 pages need no split);
// prefill_tile_body_rec below reads the step's split records instead.
// LIVE (<= TILES) is the number of tiles this wave computes; it bounds only
// the per-tile loops, never a barrier (see prefill_tile).
template <int D, typename KT, int TILES, int LIVE = TILES>
__device__ __forceinline__ void prefill_tile_body(const PrefillArgs& a, PfLds<D, KT>& sh, int bx, int by) {
    constexpr int kPrefillTiles = TILES;
    constexpr int kRow = PfLds<D, KT>::kRow;
    constexpr bool kSplitKV = sizeof(KT) == 4;  // fp32 pages enter as hi + lo pairs

    const PrefillTile t = a.tiles[bx];
    const int hc = by * kDecodeWaves * TILES;  // first head of this workgroup within the group
    const int G = min(kDecodeWaves * TILES, a.group - hc);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;  // query token of the tile (B / result column)
    const int g = lane >> 4;
    const int h0 = t.kvh * a.group + hc;
    // Tokens this lane's row attends to; padding rows past the tile get the
    // whole page range so their scores stay finite.
    const bool row_live = n < t.ntok;
    const int row_ctx = row_live ? min(t.token_count, t.pos0 + n + 1) : 0x7fffffff;

    TileQ<D> q[kPrefillTiles];
    TileState<D> st[kPrefillTiles];
#pragma unroll
    for (int s = 0; s < LIVE; ++s) {
        const int T = wave + 4 * s;
        const float* qrow = a.q + ((int64_t)(t.qi0 + (row_live ? n : 0)) * a.n_heads + h0 + (T < G ? T : 0)) * D;
        load_tile_q<D>(q[s], qrow, T < G && row_live, g, a.scale_log2);
#pragma unroll
        for (int j = 0; j < D / 16; ++j) st[s].o[j] = f4{0.f, 0.f, 0.f, 0.f};
        st[s].m = -INFINITY;
        st[s].l = 0.f;
    }

    const KT* kbase = static_cast<const KT*>(a.k_pool) + a.layer_offset + (int64_t)t.kvh * a.head_stride;
    const KT* vbase = static_cast<const KT*>(a.v_pool) + a.layer_offset + (int64_t)t.kvh * a.head_stride;
    const int32_t* bt = a.bt_ids + t.bt_base;
    const int ctx_last = min(t.token_count, t.pos0 + t.ntok);

    // Page p of the row into registers; pages past the row's last load as zeros
    // (its keys are past every row's limit, so they are masked).
    PfStage<D, KT> sr;
    auto load_regs = [&](int pg) {
        const bool have = pg < t.pages;
        const int64_t blk = have ? bt[pg] : 0;
        stage_load<D>(sr, kbase + blk * a.block_stride, vbase + blk * a.block_stride,
                      have ? min(kBlockSize, ctx_last - pg * kBlockSize) : 0);
    };
    const int pairs = (t.pages + 1) >> 1;
    load_regs(0);
    stage_store<D>(sr, sh.b[0], 0);
    load_regs(1);
    stage_store<D>(sr, sh.b[0], 1);
    __syncthreads();

    // Pages go in pairs (32 keys, one v_mfma_f32_16x16x32_f16 step of P.V).
    // The next pair is staged one page at a time: the first after this pair's
    // scores, the second at the end.
    // O is kept in units of 2^(eo - 12), eo the largest V exponent so far; it is
    // the same for every tile of the wave, which all see the same pages.
    int eo = -1000;  // below any page's V exponent: the first page sets it
    for (int i = 0; i < pairs; ++i) {
        const int buf = i & 1;
        const bool more = i + 1 < pairs;
        if (more) load_regs(2 * i + 2);
        const int key0 = i * kPairKeys + 4 * g;  // the lane's keys: key0 + r and key0 + 16 + r
        const bool diag = (i + 1) * kPairKeys > min(t.pos0 + 1, t.token_count);  // some row may stop here

        // Page scales (fp32 pages): 2^e_k and e_v of the lane's keys, and the pair's largest e_v.
        f4 ks0 = {1.f, 1.f, 1.f, 1.f}, ks1 = {1.f, 1.f, 1.f, 1.f};
        int evk[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int evmax = 0;
        if constexpr (kSplitKV) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ks0[r] = sh.b[buf].v.ks[4 * g + r];
                ks1[r] = sh.b[buf].v.ks[kBlockSize + 4 * g + r];
                evk[r] = sh.b[buf].v.ev[4 * g + r];
                evk[4 + r] = sh.b[buf].v.ev[kBlockSize + 4 * g + r];
            }
            evmax = sh.b[buf].v.evw[0];
#pragma unroll
            for (int w = 1; w < 2 * kDecodeWaves; ++w) evmax = max(evmax, sh.b[buf].v.evw[w]);
        }
        // P' = P * pv[key]: 2^(e_v(key) - eo + 12) for fp32 pages (a pair with larger
        // V exponents raises eo first, and O takes the factor eo_down), 2^12 for
        // fp16 pages.
        f4 pv0, pv1;
        bool eo_up = false;
        float eo_down = 1.f;
        if constexpr (kSplitKV) {
            if (evmax > eo) {
                eo_up = true;
                eo_down = ldexpf(1.0f, eo - evmax);  // 0 on the first pair
                eo = evmax;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pv0[r] = ldexpf(1.0f, evk[r] - eo + kPScaleLog2);
                pv1[r] = ldexpf(1.0f, evk[4 + r] - eo + kPScaleLog2);
            }
        } else {
            pv0 = f4{1.f, 1.f, 1.f, 1.f} * (float)(1 << kPScaleLog2);
            pv1 = pv0;
        }

        // S^T = K . Q^T for both pages (hi/lo products, one accumulation chain per
        // page and tile), 32 head dims per matrix-core step: A = K[key n][32j + 8g .. +7].
        // The wave's tiles share the pages, so each K operand read from LDS and
        // each V operand assembled below serves all of them.
        // The lane's parts of the LDS addresses are formed here, in every
        // iteration (the empty asm keeps them from being hoisted), so the
        // constant parts go into the instructions' immediate offsets.
        int kq = n * kRow + 8 * g;
        int vq = vt_row<kSplitKV>(4 * n) + 8 * g;
        asm volatile("" : "+v"(kq), "+v"(vq));
        f4 sc[2][kPrefillTiles];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int s = 0; s < LIVE; ++s) sc[h][s] = f4{0.f, 0.f, 0.f, 0.f};
        // Step t = 2j + h takes page h's head dims 32j .. 32j + 31; its K words
        // are read while step t - 1's products run.  Within a step the tiles'
        // chains alternate, so no product waits on the one just issued.
        auto read_k = [&](int t, h8& kh, h8& kl) {
            const int at = kq + (t & 1) * kBlockSize * kRow + 32 * (t >> 1);
            if constexpr (kSplitKV) {
                kh = *reinterpret_cast<const h8*>(&sh.b[buf].k.kh[at]);
                kl = *reinterpret_cast<const h8*>(&sh.b[buf].k.kl[at]);
            } else {
                kh = *reinterpret_cast<const h8*>(&sh.b[buf].k[at]);
            }
        };
        h8 nkh, nkl = {};
        read_k(0, nkh, nkl);
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
            const h8 kh = nkh, kl = nkl;
            if (t + 1 < D / 16) read_k(t + 1, nkh, nkl);
            __builtin_amdgcn_sched_barrier(0);  // one step's reads ahead, no more
            const int j = t >> 1, h = t & 1;
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                sc[h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, q[s].hi[j], sc[h][s], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                sc[h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, q[s].lo[j], sc[h][s], 0, 0, 0);
            if constexpr (kSplitKV) {
#pragma unroll
                for (int s = 0; s < LIVE; ++s)
                    sc[h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, q[s].hi[j], sc[h][s], 0, 0, 0);
            }
        }

        // Softmax of each tile over the pair, and its P' as an fp16 pair in the
        // A layout of the K = 32 step: elements 0..3 are the lane's keys of the
        // first page, 4..7 those of the second.
        h8 ph[kPrefillTiles], pl[kPrefillTiles];
#pragma unroll
        for (int s = 0; s < LIVE; ++s) {
            TileState<D>& ts = st[s];
            f4 p0 = sc[0][s] * q[s].sc;  // lane: S[token n][keys key0 .. key0 + 3], log2 units
            f4 p1 = sc[1][s] * q[s].sc;
            if constexpr (kSplitKV) {
                p0 *= ks0;
                p1 *= ks1;
            }
            f4 alpha_rows = {1.f, 1.f, 1.f, 1.f};
            bool rescale = false;
            pair_softmax<D>(ts, p0, p1, diag, key0, row_ctx, g, alpha_rows, rescale);

            if (eo_up) {
                alpha_rows *= eo_down;
                rescale = true;
            }
            p0 *= pv0;
            p1 *= pv1;
            if (rescale) {
#pragma unroll
                for (int b = 0; b < D / 16; ++b) ts.o[b] *= alpha_rows;
            }
            h4 h0, l0, h1, l1;
            split_pair(p0, h0, l0);
            split_pair(p1, h1, l1);
            ph[s] = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
            pl[s] = __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7);
        }

        // The first page of the next pair goes to the other buffer (free since
        // the last barrier), and its second page starts loading.
        if (more) {
            stage_store<D>(sr, sh.b[buf ^ 1], 0);
            load_regs(2 * i + 3);
        }

        // O += P' . V over the pair's 32 keys: output block b = 4c + i takes
        // B = V[keys][64c + 4n + i] for the same eight keys as the lane's P'
        // (keys 4g .. 4g + 3 of each page), one 16-byte word of the transposed
        // V.  The words of block b + 1 are read while block b's products run.
        auto read_v = [&](int b, h8& bh, h8& bl) {
            const int at = vq + vt_row<kSplitKV>(64 * (b >> 2)) + kVtStride<kSplitKV> * (b & 3);
            if constexpr (kSplitKV) {
                bh = *reinterpret_cast<const h8*>(&sh.b[buf].v.vt[at]);
                bl = *reinterpret_cast<const h8*>(&sh.b[buf].v.vt[at + kPairKeys]);
            } else {
                bh = *reinterpret_cast<const h8*>(&sh.b[buf].v[at]);
            }
        };
        h8 nbh, nbl;
        read_v(0, nbh, nbl);
#pragma unroll
        for (int b = 0; b < D / 16; ++b) {
            const h8 bh = nbh, bl = nbl;
            if (b + 1 < D / 16) read_v(b + 1, nbh, nbl);
            __builtin_amdgcn_sched_barrier(0);  // one block's reads ahead, no more
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                st[s].o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[s], bh, st[s].o[b], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                st[s].o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[s], bh, st[s].o[b], 0, 0, 0);
            if constexpr (kSplitKV) {
#pragma unroll
                for (int s = 0; s < LIVE; ++s)
                    st[s].o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[s], bl, st[s].o[b], 0, 0, 0);
            }
        }
        if (more) stage_store<D>(sr, sh.b[buf ^ 1], 1);
        __syncthreads();
    }

    // O rows are tokens 4g + r of head T; l of token n lives in lanes n (+16k).
#pragma unroll
    for (int s = 0; s < LIVE; ++s) {
        const int T = wave + 4 * s;
        if (T >= G) continue;
        float ls = st[s].l;
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        const float unit = ldexpf(1.0f, (kSplitKV ? eo : 0) - kPScaleLog2);
        f4 inv;
#pragma unroll
        for (int r = 0; r < 4; ++r) inv[r] = unit / __shfl(ls, 4 * g + r);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = 4 * g + r;
            if (tok < t.ntok) {
                float* orow = a.out + ((int64_t)(t.qi0 + tok) * a.n_heads + h0 + T) * D;
#pragma unroll
                for (int c = 0; c < D / 64; ++c) {
                    f4 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = st[s].o[4 * c + i][r] * inv[r];
                    *reinterpret_cast<f4*>(orow + 64 * c + 4 * n) = v;
                }
            }
        }
    }
}

// Records form, software-pipelined.  Iteration k runs the score products of
// pair k while the same wave's vector ALUs run the softmax of pair k - 1 (two
// independent instruction streams, interleaved below so that the vector work
// issues while the matrix cores run), then the P.V products of pair k - 1.
// K and V halves have their own double buffers: iteration k reads K(k) and
// V(k - 1) and loads K(k + 1) and V(k) behind them, so LDS holds four halves,
// the two buffers of the form above.  The arithmetic is that of
// prefill_tile_body; the softmax is written without branches, the rare O
// rescale being the one branch, between the two groups of products.
template <int D>
struct alignas(16) PfLdsPipe {
    PfKHalf<D> k[2];
    PfVHalf<D> v[2];
};

// Largest of eight floats and of a row's four lane groups, without the
// quieting that fmaxf adds to loaded values (scores are never NaN here).
__device__ __forceinline__ float max8(const f4& a, const f4& b) {
    float m;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(m) : "v"(a[0]), "v"(a[1]), "v"(a[2]));
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(m) : "v"(m), "v"(a[3]), "v"(b[0]));
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(m) : "v"(m), "v"(b[1]), "v"(b[2]));
    asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(m), "v"(b[3]));
    return m;
}

__device__ __forceinline__ float cross_row_max_raw(float x) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    asm("v_max_f32 %0, %1, %2" : "=v"(x) : "v"(__uint_as_float(r16[0])), "v"(__uint_as_float(r16[1])));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    asm("v_max_f32 %0, %1, %2" : "=v"(x) : "v"(__uint_as_float(r32[0])), "v"(__uint_as_float(r32[1])));
    return x;
}

// pair_softmax of raw scores s (their log2-unit value is t = s * c, c > 0:
// the tile's Q carries the scale's sign), without branches or lane exchanges
// beyond the row max: m moves for every lane when some row of the wave grew
// by more than kLazyLog2 (`grew`); alpha is token n's factor (1 where m did
// not move), which the O rows take only when something grew.  P = 2^(t - m)
// with t rounded first: m is a rounded t, so the largest score gives exactly
// 2^0 however large the scores are (a fused s * c - m would keep up to half an
// ulp of t, which for scores near 2^40 overflows exp2).
template <bool MASK>
__device__ __forceinline__ void pair_softmax_rec(float& m, float& l, f4& s0, f4& s1, float c, int key0, int row_ctx,
                                                 float& alpha, bool& grew) {
    // No multiply-add contraction here: the max and the exponents must see the
    // same rounded scores (a fused s * c - m keeps the product unrounded).
#pragma clang fp contract(off)
    if constexpr (MASK) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s0[r] = key0 + r >= row_ctx ? -INFINITY : s0[r];
            s1[r] = key0 + kBlockSize + r >= row_ctx ? -INFINITY : s1[r];
        }
    }
    s0 *= c;
    s1 *= c;
    const float mp = cross_row_max_raw(max8(s0, s1));
    grew = __any(mp > m + kLazyLog2);  // true on the first pair (m = -inf)
    const float mn = grew ? fmaxf(m, mp) : m;  // finite: the first pair holds key 0 for every row
    alpha = fast_exp2(m - mn);  // 1 where m stays, 0 on the first pair
    m = mn;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s0[r] = fast_exp2(s0[r] - mn);
        s1[r] = fast_exp2(s1[r] - mn);
    }
    l = l * alpha + (((s0[0] + s0[1]) + (s0[2] + s0[3])) + ((s1[0] + s1[1]) + (s1[2] + s1[3])));
}

// LIVE bounds only the per-tile loops, never a barrier (see prefill_tile).
template <int D, int TILES, int LIVE = TILES>
__device__ __forceinline__ void prefill_tile_body_rec(const PrefillArgs& a, PfLdsPipe<D>& sh, int bx, int by) {
    constexpr int kRow = D + 8;
    constexpr int kSteps = D / 16;  // score steps per pair (32 head dims of one page each), = output blocks
    const PrefillTile t = a.tiles[bx];
    const int hc = by * kDecodeWaves * TILES;
    const int G = min(kDecodeWaves * TILES, a.group - hc);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;
    const int g = lane >> 4;
    const int h0 = t.kvh * a.group + hc;
    const bool row_live = n < t.ntok;
    const int row_ctx = row_live ? min(t.token_count, t.pos0 + n + 1) : 0x7fffffff;

    // Pair i of the tile is record t.rec0 + i.
    const int pairs = (t.pages + 1) >> 1;
    auto record = [&](int i) {
        return prefill_rsrc(a.records + ((int64_t)t.rec0 + i) * kRecordBytes<D>, kRecordBytes<D>);
    };
    auto load_k = [&](int i) { half_load<D>(&sh.k[i & 1], record(i), 0); };
    auto load_v = [&](int i) { half_load<D>(&sh.v[i & 1], record(i), kHalfBytes<D>); };
    load_k(0);

    TileQ<D> q[TILES];
    TileState<D> st[TILES];
#pragma unroll
    for (int s = 0; s < LIVE; ++s) {
        const int T = wave + 4 * s;
        const float* qrow = a.q + ((int64_t)(t.qi0 + (row_live ? n : 0)) * a.n_heads + h0 + (T < G ? T : 0)) * D;
        load_tile_q<D>(q[s], qrow, T < G && row_live, g, a.scale_log2);
#pragma unroll
        for (int j = 0; j < kSteps; ++j) st[s].o[j] = f4{0.f, 0.f, 0.f, 0.f};
        st[s].m = -INFINITY;
        st[s].l = 0.f;
    }
    const int kq = n * kRow + 8 * g;              // the lane's K word in a K half (halves)
    const int vq = vt_row<true>(4 * n) + 8 * g;   // its V word in a V half

    // S^T = K . Q^T of pair i for every tile: step u takes page u & 1's head
    // dims 32 (u >> 1) .. + 31; the tiles' chains alternate within a step.
    auto scores = [&](int i, f4 (&sc)[2][TILES]) {
        const _Float16* kh = sh.k[i & 1].kh;
        const _Float16* kl = sh.k[i & 1].kl;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int s = 0; s < LIVE; ++s) sc[h][s] = f4{0.f, 0.f, 0.f, 0.f};
        auto read_k = [&](int u, h8& khv, h8& klv) {
            const int at = kq + (u & 1) * kBlockSize * kRow + 32 * (u >> 1);
            khv = *reinterpret_cast<const h8*>(&kh[at]);
            klv = *reinterpret_cast<const h8*>(&kl[at]);
        };
        h8 nkh, nkl;
        read_k(0, nkh, nkl);
#pragma unroll
        for (int u = 0; u < kSteps; ++u) {
            const h8 khv = nkh, klv = nkl;
            if (u + 1 < kSteps) read_k(u + 1, nkh, nkl);
            __builtin_amdgcn_sched_barrier(0);  // one step's reads ahead, no more
            const int j = u >> 1, h = u & 1;
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                sc[h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khv, q[s].hi[j], sc[h][s], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                sc[h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khv, q[s].lo[j], sc[h][s], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                sc[h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(klv, q[s].hi[j], sc[h][s], 0, 0, 0);
        }
    };

    // The scales of pair i, from its V half: the pair's one K factor (records
    // carry one K exponent per pair) and the V exponents of the lane's eight keys.
    struct PairScales {
        float ks;
        int evk[8];
        int evw[2 * kDecodeWaves];
    };
    auto read_scales = [&](int i, PairScales& ps) {
        const PfVHalfBody<D>& vb = sh.v[i & 1];
        ps.ks = vb.ks[0];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ps.evk[r] = vb.ev[4 * g + r];
            ps.evk[4 + r] = vb.ev[kBlockSize + 4 * g + r];
        }
#pragma unroll
        for (int w = 0; w < 2 * kDecodeWaves; ++w) ps.evw[w] = vb.evw[w];
    };

    // Softmax of pair i (its scores in sc) for every tile, into P' as fp16
    // pairs; need[s]: tile s's O rows must take alpha[s] (token n's factor) and
    // eo_down before P'.V is added.
    int eo = -1000;  // O is kept in units of 2^(eo - 12), eo the largest V exponent so far
    float eo_down = 1.f;
    auto softmax = [&](auto masked, int i, f4 (&sc)[2][TILES], const PairScales& ps, h8 (&ph)[TILES],
                       h8 (&pl)[TILES], float (&alpha)[TILES], bool (&need)[TILES]) {
        const float ks = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ps.ks)));  // one per pair
        const int* evk = ps.evk;
        int evmax = ps.evw[0];
#pragma unroll
        for (int w = 1; w < 2 * kDecodeWaves; ++w) evmax = max(evmax, ps.evw[w]);
        const bool eo_up = evmax > eo;
        eo_down = ldexpf(1.0f, min(0, eo - evmax));  // 0 on the first pair
        eo = max(eo, evmax);
        f4 pv0, pv1;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pv0[r] = ldexpf(1.0f, evk[r] - eo + kPScaleLog2);
            pv1[r] = ldexpf(1.0f, evk[4 + r] - eo + kPScaleLog2);
        }
        const int key0 = i * kPairKeys + 4 * g;
#pragma unroll
        for (int s = 0; s < LIVE; ++s) {
            f4 p0 = sc[0][s];
            f4 p1 = sc[1][s];
            bool grew;
            pair_softmax_rec<decltype(masked)::value>(st[s].m, st[s].l, p0, p1, q[s].sc * ks, key0, row_ctx, alpha[s],
                                                      grew);
            need[s] = grew || eo_up;
            p0 *= pv0;
            p1 *= pv1;
            h4 hi0, lo0, hi1, lo1;
            split_pair(p0, hi0, lo0);
            split_pair(p1, hi1, lo1);
            ph[s] = __builtin_shufflevector(hi0, hi1, 0, 1, 2, 3, 4, 5, 6, 7);
            pl[s] = __builtin_shufflevector(lo0, lo1, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };

    // O += P'.V over pair i: block b takes B = V[keys][64 (b >> 2) + 4 n + (b & 3)].
    auto values = [&](int i, const h8 (&ph)[TILES], const h8 (&pl)[TILES]) {
        const _Float16* vt = sh.v[i & 1].vt;
        auto read_v = [&](int b, h8& bh, h8& bl) {
            const int at = vq + vt_row<true>(64 * (b >> 2)) + kVtStride<true> * (b & 3);
            bh = *reinterpret_cast<const h8*>(&vt[at]);
            bl = *reinterpret_cast<const h8*>(&vt[at + kPairKeys]);
        };
        h8 nbh, nbl;
        read_v(0, nbh, nbl);
#pragma unroll
        for (int b = 0; b < kSteps; ++b) {
            const h8 bh = nbh, bl = nbl;
            if (b + 1 < kSteps) read_v(b + 1, nbh, nbl);
            __builtin_amdgcn_sched_barrier(0);  // one block's reads ahead, no more
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                st[s].o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[s], bh, st[s].o[b], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                st[s].o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[s], bh, st[s].o[b], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < LIVE; ++s)
                st[s].o[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[s], bl, st[s].o[b], 0, 0, 0);
        }
    };

    // O rows are tokens 4g + r: their factors come from the lanes of those tokens.
    auto rescale = [&](const float (&alpha)[TILES], const bool (&need)[TILES]) {
#pragma unroll
        for (int s = 0; s < LIVE; ++s) {
            if (need[s]) {
                f4 rows;
#pragma unroll
                for (int r = 0; r < 4; ++r) rows[r] = __shfl(alpha[s], 4 * g + r) * eo_down;
#pragma unroll
                for (int b = 0; b < kSteps; ++b) st[s].o[b] *= rows;
            }
        }
    };

    record_wait();
    __syncthreads();
    if (pairs > 1) load_k(1);
    load_v(0);
    f4 sa[2][TILES], sb[2][TILES];  // scores of the pair before the current one, and of the current one
    scores(0, sa);
    record_wait();
    __syncthreads();

    // Iteration k: scores of pair k into sout while the softmax of pair k - 1
    // (scores in sin) runs, then P'.V of pair k - 1.  Pair i needs the causal
    // mask when some row of the tile may stop inside it.
    const int first_diag = min(pairs, min(t.pos0 + 1, t.token_count) / kPairKeys);
    auto iteration = [&](auto masked, int k, f4 (&sin)[2][TILES], f4 (&sout)[2][TILES]) {
        if (k + 1 < pairs) load_k(k + 1);
        load_v(k);
        h8 ph[TILES], pl[TILES];
        float alpha[TILES];
        bool need[TILES];
        PairScales ps;
        read_scales(k - 1, ps);
        scores(k, sout);
        softmax(masked, k - 1, sin, ps, ph, pl, alpha, need);
        rescale(alpha, need);
        values(k - 1, ph, pl);
        record_wait();
        __syncthreads();
    };
    int k = 1;
    for (const int k_plain = min(pairs, first_diag + 1); k < k_plain; ++k) {
        iteration(std::false_type{}, k, sa, sb);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int s = 0; s < LIVE; ++s) sa[h][s] = sb[h][s];
    }
    for (; k < pairs; ++k) {
        iteration(std::true_type{}, k, sa, sb);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int s = 0; s < LIVE; ++s) sa[h][s] = sb[h][s];
    }
    {
        h8 ph[TILES], pl[TILES];
        float alpha[TILES];
        bool need[TILES];
        PairScales ps;
        read_scales(pairs - 1, ps);
        softmax(std::true_type{}, pairs - 1, sa, ps, ph, pl, alpha, need);
        rescale(alpha, need);
        values(pairs - 1, ph, pl);
    }

    // O rows are tokens 4g + r of head T; l of token n lives in lanes n (+16k).
#pragma unroll
    for (int s = 0; s < LIVE; ++s) {
        const int T = wave + 4 * s;
        if (T >= G) continue;
        float ls = st[s].l;
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        const float unit = ldexpf(1.0f, eo - kPScaleLog2);
        f4 inv;
#pragma unroll
        for (int r = 0; r < 4; ++r) inv[r] = unit / __shfl(ls, 4 * g + r);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = 4 * g + r;
            if (tok < t.ntok) {
                float* orow = a.out + ((int64_t)(t.qi0 + tok) * a.n_heads + h0 + T) * D;
#pragma unroll
                for (int c = 0; c < D / 64; ++c) {
                    f4 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = st[s].o[4 * c + i][r] * inv[r];
                    *reinterpret_cast<f4*>(orow + 64 * c + 4 * n) = v;
                }
            }
        }
    }
}

// Runs tile workgroup (bx, by) of either body.  With two tiles per wave, a
// wave whose second head is past the group (wave + 4 >= G: groups of 5 to 7
// heads, or a partial last head chunk) computes its first tile only; its
// barriers and copies are the same, so the workgroup stays in step.  The
// waves of one workgroup then run different instantiations (LIVE = 1 and
// LIVE = TILES), which is correct only because LIVE bounds nothing but the
// unrolled per-tile loops of straight-line arithmetic: every barrier, LDS
// copy and page load of the bodies sits outside those loops and runs the same
// number of times in both.  Keep it so: a barrier inside a LIVE-bounded loop
// would leave the workgroup's waves at different barriers.  Skipping
// the padding tile's products took a Qwen2.5-7B-shape batch of sixteen prefill
// chunks (group 7) from 268-273 us to 260-263 us.
template <int D, typename KT, int TILES, bool REC, typename Sh>
__device__ __forceinline__ void prefill_tile(const PrefillArgs& a, Sh& sh, int bx, int by) {
    const int G = min(kDecodeWaves * TILES, a.group - by * kDecodeWaves * TILES);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool one = TILES == 2 && wave + kDecodeWaves >= G;
    if constexpr (REC) {
        if (one) prefill_tile_body_rec<D, TILES, 1>(a, sh, bx, by);
        else prefill_tile_body_rec<D, TILES>(a, sh, bx, by);
    } else {
        if (one) prefill_tile_body<D, KT, TILES, 1>(a, sh, bx, by);
        else prefill_tile_body<D, KT, TILES>(a, sh, bx, by);
    }
}

template <int D, typename KT, int TILES, bool REC>
__global__ __launch_bounds__(kDecodeThreads, 2) void paged_prefill_mfma_kernel(PrefillArgs a) {
    if constexpr (REC) {
        __shared__ PfLdsPipe<D> sh;
        prefill_tile<D, KT, TILES, true>(a, sh, blockIdx.x, blockIdx.y);
    } else {
        __shared__ PfLds<D, KT> sh;
        prefill_tile<D, KT, TILES, false>(a, sh, blockIdx.x, blockIdx.y);
    }
}

// A step with both decode units and prefill tiles in one launch: workgroups
// x < num_bins run decode bin x (decode_bins_body, grid.y = its tiles of 16
// heads), the others prefill tile x - num_bins (grid.y = its groups of 4 TILES
// heads); a workgroup past its kind's grid.y returns at once.  The decode
// workgroups come first, so each is dispatched onto a CU whose other slot
// takes a tile: HBM-bound and matrix-bound waves share the CUs in one kernel,
// with no second stream (streams share the device's few hardware queues, and
// two kernels on one queue run one after the other).
template <int D, typename KT, int TILES, bool REC>
__global__ __launch_bounds__(kDecodeThreads, 2) void paged_mixed_mfma_kernel(DecodeArgs da, PrefillArgs pa, int num_bins,
                                                                          int decode_y, int tile_y) {
    __shared__ union {
        EpilogueLds<D, kMaxGroupMfma> d;
        typename std::conditional<REC, PfLdsPipe<D>, PfLds<D, KT>>::type p;
    } sh;
    const int bx = blockIdx.x;
    const int by = blockIdx.y;
    if (bx < num_bins) {
        if (by < decode_y) decode_bins_body<D, KT, kExact>(da, sh.d, bx, by);
    } else if (by < tile_y) {
        prefill_tile<D, KT, TILES, REC>(pa, sh.p, bx - num_bins, by);
    }
}

template <int D, typename KT>
hipError_t launch_mixed(int num_bins, int num_tiles, const DecodeArgs& da, const PrefillArgs& pa, hipStream_t stream) {
    const int tiles = pa.group > kDecodeWaves ? 2 : 1;
    const int per_wg = kDecodeWaves * tiles;
    const int decode_y = (da.group + kDecodeTileHeads - 1) / kDecodeTileHeads;
    const int tile_y = (pa.group + per_wg - 1) / per_wg;
    const dim3 grid(num_bins + num_tiles, max(decode_y, tile_y));
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(kDecodeThreads), 0, stream, da, pa, num_bins, decode_y, tile_y);
    };
    if constexpr (sizeof(KT) == 4) {
        if (pa.records) {
            if (tiles == 2) go(paged_mixed_mfma_kernel<D, KT, 2, true>);
            else go(paged_mixed_mfma_kernel<D, KT, 1, true>);
            return hipGetLastError();
        }
    }
    if (tiles == 2) go(paged_mixed_mfma_kernel<D, KT, 2, false>);
    else go(paged_mixed_mfma_kernel<D, KT, 1, false>);
    return hipGetLastError();
}

template <int D, typename KT>
hipError_t launch_tiles(int num_tiles, const PrefillArgs& a, hipStream_t stream) {
    const int tiles = a.group > kDecodeWaves ? 2 : 1;
    const int per_wg = kDecodeWaves * tiles;
    static_assert(kPrefillHeads == 2 * kDecodeWaves, "a workgroup covers at most kPrefillHeads heads");
    const dim3 grid(num_tiles, (a.group + per_wg - 1) / per_wg);
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kDecodeThreads), 0, stream, a); };
    if constexpr (sizeof(KT) == 4) {
        if (a.records) {
            if (tiles == 2) go(paged_prefill_mfma_kernel<D, KT, 2, true>);
            else go(paged_prefill_mfma_kernel<D, KT, 1, true>);
            return hipGetLastError();
        }
    }
    if (tiles == 2) go(paged_prefill_mfma_kernel<D, KT, 2, false>);
    else go(paged_prefill_mfma_kernel<D, KT, 1, false>);
    return hipGetLastError();
}

}  // namespace

int prefill_record_bytes(int head_dim) {
    return head_dim == 128 ? kRecordBytes<128> : head_dim == 64 ? kRecordBytes<64> : 0;
}

hipError_t launch_prefill_split(int head_dim, int num_items, int max_pairs, const PrefillSplitArgs& a,
                                hipStream_t stream) {
    if (num_items <= 0 || max_pairs <= 0) return hipSuccess;
    if (!a.records || !a.items || num_items > 65535) return hipErrorInvalidValue;
    const dim3 grid(max_pairs, num_items);
    if (head_dim == 128) hipLaunchKernelGGL(prefill_split_kernel<128>, grid, dim3(kDecodeThreads), 0, stream, a);
    else if (head_dim == 64) hipLaunchKernelGGL(prefill_split_kernel<64>, grid, dim3(kDecodeThreads), 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_mixed_mfma(int head_dim, int kv_f16, int num_bins, int num_tiles, const DecodeArgs& da,
                             const PrefillArgs& pa, hipStream_t stream) {
    if (num_bins <= 0 || num_tiles <= 0 || da.group < 1 || pa.group != da.group) return hipErrorInvalidValue;
    if (kv_f16 && pa.records) return hipErrorInvalidValue;
    if (da.head_dim != head_dim || da.v_head_dim != head_dim || da.block_size != kBlockSize || da.tile_pages != 1)
        return hipErrorInvalidValue;
    if (head_dim == 128) return kv_f16 ? launch_mixed<128, _Float16>(num_bins, num_tiles, da, pa, stream)
                                       : launch_mixed<128, float>(num_bins, num_tiles, da, pa, stream);
    if (head_dim == 64) return kv_f16 ? launch_mixed<64, _Float16>(num_bins, num_tiles, da, pa, stream)
                                      : launch_mixed<64, float>(num_bins, num_tiles, da, pa, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_prefill_mfma(int head_dim, int kv_f16, int num_tiles, const PrefillArgs& a, hipStream_t stream) {
    if (num_tiles <= 0) return hipSuccess;
    if (a.group < 1 || (kv_f16 && a.records)) return hipErrorInvalidValue;
    if (head_dim == 128) return kv_f16 ? launch_tiles<128, _Float16>(num_tiles, a, stream)
                                       : launch_tiles<128, float>(num_tiles, a, stream);
    if (head_dim == 64) return kv_f16 ? launch_tiles<64, _Float16>(num_tiles, a, stream)
                                      : launch_tiles<64, float>(num_tiles, a, stream);
    return hipErrorInvalidValue;
}

}  // namespace gsp
