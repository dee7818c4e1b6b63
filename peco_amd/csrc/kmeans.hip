// Stage 1: batched Lloyd k-means over Q and K per (batch, head), for gfx950.
//
// Reference semantics (peco/clustering.py:45-89, CPU branch; tie rule kmeans.cu:43,55-56):
//   label[t] = argmin_j ( -2 x_t.c_j + |c_j|^2 ), lowest j on ties
//   mean[j]  = (sum of member rows) / count, or the previous centre when empty.
// The fp32 order is fixed so results are reproducible bit for bit:
//   n_j   = sum_d fl(c_jd^2), d ascending                      (centre norm)
//   D_tj  = fma(-2, dot_tj, n_j), dot_tj = fma chain, d ascending
//   sum_j = fp32 adds of member rows in original token order   (== torch scatter_add_)
//
// Assignment never evaluates D_tj for every pair. A bf16 MFMA screen computes
//   S_tj = |c_j|^2 + x_t . (c_hi + c_lo)*(-2)   with c_hi = bf16(c), c_lo = bf16(c - c_hi)
// (x itself is split the same way when it is not bf16), whose error against the canonical
// distance is bounded a priori (|c - c_hi - c_lo| <= 2^-16 |c|, products exact in fp32,
// fp32 accumulation error <= gamma_n, canonical chain error <= gamma_D). Each token keeps
// its three smallest screened values with the centre index packed into the low mantissa
// bits. With best and second best b1 <= b2 and the bound E, b2 - b1 > 2E proves that the
// centre of b1 is the canonical argmin. Otherwise every centre screening within b1 + 2E is
// a candidate (all of them are among the kept three unless that list is saturated); the
// candidates get the canonical fp32 distance in-kernel, lowest index on ties, and a
// saturated list falls back to evaluating all centres. Labels are therefore identical to the
// canonical fixed-order fp32 definition, not approximately equal.
//
// Per iteration: assign (+ per-tile label histogram via global atomics) -> sort scan ->
// sort place (stable counting sort, also yields the final permutation for stage 3) ->
// update (sequential per-cluster sums in token order; also prepares the next iteration's
// split-bf16 centres and canonical norms). The problems' heads run as four chains of launches
// on four streams (km_fit_chains), or share every launch when no side stream is available.
#include "base_offset.hpp"
#include "common.hpp"
#include "sort.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <mutex>
#include <vector>

namespace peco {

struct KmProblem {
    const void* x;          // [batch, tokens, D] rows (dtype of the fit); batch stride x_stride
    int64_t x_stride;       // elements between consecutive batch entries of x (>= tokens * D)
    const float* centers_in;  // [batch, K, D] initial centres (read only)
    float* centers_out;     // [batch, K, D] final centres
    float* centers_tmp;     // [batch, K, D] ping-pong buffer
    int32_t* labels;        // [batch, tokens]
    int32_t* counts;        // [batch, K]
    int32_t* indices;       // [batch, tokens] stable sort of the final labels
    int32_t* offsets;       // [batch, K + 1]
    uint16_t* prep_hi;      // [batch, K, D] bf16(-2 c)
    uint16_t* prep_lo;      // [batch, K, D] bf16(-2 c - hi)
    float* norms;           // [batch, K] canonical norms of the current centres
    int32_t* tile_hist;     // [batch, sort tiles, K] (cleared by the prep kernel)
    int32_t* tile_hist2;    // nullable second histogram set: alternates with tile_hist per iteration
    float* sums;            // nullable [batch, K, D]: per-cluster sums of the last update
    float* xsq;             // nullable [batch, tokens]: squared token norms (certification bound),
                            // written by the first assign of a fit and read by the later ones
    int batch, tokens, clusters;
    int assign_begin;       // first linear assign block of this problem
    int assign_blocks;      // batch * ceil(tokens / kAssignTile)
    int update_begin;       // first linear prep block (batch * K blocks)
    int scan_begin;         // first linear update workgroup (batch * ceil(K / 8))
    int scan_blocks;
    int sort_tiles;
    int upd_begin;          // first linear km_update_kernel workgroup of this problem
    int upd_blocks;
    int upd_shared;         // 1: one workgroup per cluster, 0: one wavefront per cluster
    int pack_begin;         // first linear km_pack_rows_kernel workgroup (hat_order 1 only)
    int pack_blocks;        // batch * ceil(length / rows per packing workgroup)
    // Packing by the last update (nullable hat): rows [0, tokens) of hat [batch, length, D]
    // receive x's rows in cluster order, Base-Offset fake-quantized (hat_bits) against the
    // final centres, and rows [tokens, length) x's own rows past `tokens` (text, in the same
    // batch stride); with_in/with_out (nullable, [batch, length, D]) are gathered alike
    // without quantization. codes/low/scale (nullable together, [batch, tokens, D] uint8 and
    // [batch, tokens] fp32) receive the packed rows' Base-Offset payload in the same order.
    // hat_order 1 writes every row at its own token position instead (original order; no
    // with_in/with_out then), so hat is x with its video rows fake-quantized: a token-parallel
    // launch after the last update (km_pack_rows_kernel) rather than the update's own pass.
    void* hat;
    const void* with_in;
    void* with_out;
    uint8_t* codes;
    float* low;
    float* scale;
    int hat_bits;
    int length;
    int hat_order;
};

constexpr int kMaxKm = 2;
constexpr int kAssignWaves = 4;                    // wavefronts per assign workgroup
constexpr int kAssignThreads = kAssignWaves * 64;
constexpr int kAssignTile = kAssignWaves * 64;      // tokens per assign workgroup (64 per wave)

struct KmArgs {
    KmProblem p[kMaxKm];
    int num;
    int total_assign_blocks;
    int total_update_blocks;
    int total_scan_blocks;
    int total_upd_blocks;
    int text_blocks;  // packing launch only: workgroups after the update's that copy text rows
    int total_pack_blocks;  // km_pack_rows_kernel grid (problems packed in original order)
    float kappa;      // bound coefficient: |screened - canonical| <= kappa*|x||c| + rounding terms
    float gamma_acc;  // gamma of the MFMA accumulation length (applied to the norm term)
};

struct KmIter {
    const float* src[kMaxKm];  // centres used by this iteration
    float* dst[kMaxKm];        // means written by this iteration
    int32_t* hist[kMaxKm];     // nullable: tile histograms the assign adds its labels to
    float* screen;             // kDump assignments only: screened distances [batch, tokens, K]
    int sq_mode;               // token norms: 0 computed by the assign, 1 computed and stored to
                               // P.xsq, 2 read from P.xsq (x is the same in every iteration)
};

namespace {

__device__ __forceinline__ int km_problem(const KmArgs& a, int block, bool assign) {
    int p = 0;
    if (assign) {
        // Assign blocks are laid out largest-K problem first (longest blocks dispatched first).
        while (p + 1 < a.num && !(block >= a.p[p].assign_begin && block < a.p[p].assign_begin + a.p[p].assign_blocks)) ++p;
    } else {
        while (p + 1 < a.num && block >= a.p[p + 1].update_begin) ++p;
    }
    return p;
}

__device__ __forceinline__ int km_scan_problem(const KmArgs& a, int block) {
    int p = 0;
    while (p + 1 < a.num && !(block >= a.p[p].scan_begin && block < a.p[p].scan_begin + a.p[p].scan_blocks)) ++p;
    return p;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u16x8 u) { return __builtin_bit_cast(bf16x8, u); }

// Canonical norm and split-bf16 preparation of one centre row held in LDS.
__device__ __forceinline__ float canonical_norm_lds(const float* row, int D) {
    float s = 0.0f;
    for (int d = 0; d < D; ++d) {
        const float sq = row[d] * row[d];
        s = s + sq;
    }
    return s;
}

__device__ __forceinline__ void split_neg2(float c, uint16_t& hi, uint16_t& lo) {
    const float v = -2.0f * c;
    hi = f32_to_bf16_bits(v);
    lo = f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
}

// Initial preparation: norms + split of the initial centres (when the problem has split
// buffers); clears the tile histograms.
template <int D>
__global__ __launch_bounds__(64) void km_prep_kernel(KmArgs a, KmIter it) {
    __shared__ float row[D];
    int p = 0;
    int block = blockIdx.x;
    while (p + 1 < a.num && block >= a.p[p + 1].update_begin) ++p;
    const KmProblem& P = a.p[p];
    const int local = block - P.update_begin;  // b * K + j
    const float* c = it.src[p] + static_cast<int64_t>(local) * D;
    for (int d = threadIdx.x; d < D; d += kWave) {
        const float v = c[d];
        row[d] = v;
        if (P.prep_hi) {
            uint16_t hi, lo;
            split_neg2(v, hi, lo);
            P.prep_hi[static_cast<int64_t>(local) * D + d] = hi;
            P.prep_lo[static_cast<int64_t>(local) * D + d] = lo;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) P.norms[local] = canonical_norm_lds(row, D);
    // Clear this problem's tile histograms (strided over the problem's blocks), when it has them.
    if (!P.tile_hist) return;
    const int64_t hist = static_cast<int64_t>(P.batch) * P.sort_tiles * P.clusters;
    const int64_t nblocks = static_cast<int64_t>(P.batch) * P.clusters;
    for (int64_t i = static_cast<int64_t>(local) * kWave + threadIdx.x; i < hist; i += nblocks * kWave)
        P.tile_hist[i] = 0;
}

// x operand (B of the MFMA): 8 consecutive channels of one token. bf16 rows are loaded raw
// first, so every row load of a tile is in flight before any of them is used.
template <int DT> struct XChunk { u16x8 u; };

template <int DT>
__device__ __forceinline__ XChunk<DT> load_x8(const void* x, int64_t e) {
    return XChunk<DT>{*reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(x) + e)};
}

// fp16/fp32 rows: load and split one chunk (hi, lo) in place; zero for an invalid token.
template <int DT, bool kSq = true>
__device__ __forceinline__ void load_split_x8(const void* x, int64_t e, bool valid, u16x8& hi, u16x8& lo, float& sq) {
    if (!valid) {
        hi = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        lo = hi;
        return;
    }
    float f[8];
    if constexpr (DT == kF32) {
        const f32x4 a = reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + e)[0];
        const f32x4 b = reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + e)[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) { f[i] = a[i]; f[4 + i] = b[i]; }
    } else {
        const u16x8 u = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(x) + e);
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = f16_bits_to_f32(u[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint16_t h = f32_to_bf16_bits(f[i]);
        hi[i] = h;
        lo[i] = f32_to_bf16_bits(f[i] - bf16_bits_to_f32(h));
        if constexpr (kSq) sq = fmaf(f[i], f[i], sq);
    }
}

// bf16 rows: hi is the raw chunk and lo zero. An invalid token's chunk (a copy of the last row,
// loaded clamped) is used as it is: its screened values are never read. With kSq the squares of
// a valid token's chunk are added to sq.
template <int DT, bool kSq = true>
__device__ __forceinline__ void split_x8(const XChunk<DT>& r, bool valid, u16x8& hi, u16x8& lo, float& sq) {
    static_assert(DT == kBF16, "split_x8 handles bf16 rows");
    hi = r.u;
    lo = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if constexpr (kSq) {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float f = bf16_bits_to_f32(r.u[i]);
            part = fmaf(f, f, part);
        }
        sq += valid ? part : 0.0f;
    }
}

// Assign: one workgroup = kAssignTile tokens of one (problem, batch); wave w owns tokens
// [64w, 64w+64) as two 32-token MFMA column blocks (two-wave workgroups, four per CU,
// measured no faster). Centres stream through LDS in blocks of
// 32 (split-bf16 hi/lo rows + canonical norms), double-buffered with a register prefetch.
// MFMA 32x32x16: A = centres (32 rows x 16 channels), B = tokens (16 channels x 32 tokens);
// lane l holds token l%32 of each column block and centres 8*(i/4)+4*(l/32)+i%4.
// Screened distance of centres past K (finite, so index bits can be packed into it).
constexpr float kFarAway = 1.0e37f;
// Screened values kept per token and lane half (candidates for the canonical recheck).
constexpr int kTop = 3;
// VALU instructions of the candidate tracking placed after each screen MFMA.
constexpr int kTrackValuPerMfma = 5;

template <int D> struct AssignTiles {
    static constexpr int kRow = D + 8;                 // padded LDS row (16-bit elements)
    static constexpr int kElems = 32 * kRow;
    static constexpr int kChunks = D / 8;              // 16-byte chunks per row
    static constexpr int kLoads = 32 * kChunks / kAssignThreads;  // 16-byte loads per thread per array
};

template <int D> struct CentreRegs {
    u32x4 hi[AssignTiles<D>::kLoads], lo[AssignTiles<D>::kLoads];
    float norm;
};

// kRaw: the split planes are made here from the fp32 centres (raw), so a caller needs no
// buffer for them; otherwise they are read from hi_base/lo_base.
template <int D, bool kRaw>
__device__ __forceinline__ void load_centres(CentreRegs<D>& R, const uint16_t* hi_base, const uint16_t* lo_base,
                                             const float* raw, const float* norms, int cb, int K, int tid) {
    using T = AssignTiles<D>;
#pragma unroll
    for (int i = 0; i < T::kLoads; ++i) {
        const int id = i * kAssignThreads + tid;
        const int row = min(cb + id / T::kChunks, K - 1);  // rows past K are never selected
        const int64_t e = static_cast<int64_t>(row) * D + (id % T::kChunks) * 8;
        if constexpr (kRaw) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(raw + e);
            const f32x4 b = *reinterpret_cast<const f32x4*>(raw + e + 4);
            uint16_t h[8], l[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                split_neg2(a[k], h[k], l[k]);
                split_neg2(b[k], h[4 + k], l[4 + k]);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                R.hi[i][k] = static_cast<uint32_t>(h[2 * k]) | (static_cast<uint32_t>(h[2 * k + 1]) << 16);
                R.lo[i][k] = static_cast<uint32_t>(l[2 * k]) | (static_cast<uint32_t>(l[2 * k + 1]) << 16);
            }
        } else {
            R.hi[i] = *reinterpret_cast<const u32x4*>(hi_base + e);
            R.lo[i] = *reinterpret_cast<const u32x4*>(lo_base + e);
        }
    }
    if (tid < 32) R.norm = cb + tid < K ? norms[cb + tid] : kFarAway;
}

template <int D>
__device__ __forceinline__ void store_centres(const CentreRegs<D>& R, uint16_t* hi, uint16_t* lo, float* nrm, int tid) {
    using T = AssignTiles<D>;
#pragma unroll
    for (int i = 0; i < T::kLoads; ++i) {
        const int id = i * kAssignThreads + tid;
        const int off = (id / T::kChunks) * T::kRow + (id % T::kChunks) * 8;
        *reinterpret_cast<u32x4*>(hi + off) = R.hi[i];
        *reinterpret_cast<u32x4*>(lo + off) = R.lo[i];
    }
    if (tid < 32) nrm[tid] = R.norm;
}

// Canonical dot x_t . c_j: fma chain over d ascending (the oracle's order). Loads go out
// 32 channels at a time so a dot costs D/32 memory latencies, not D.
template <int DT, int D>
__device__ __forceinline__ float canonical_dot(const void* x, int64_t xrow, const float* c) {
    float dot = 0.0f;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += 32) {
        float xv[32], cv[32];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float tmp[8];
            if constexpr (DT == kF32) {
                const f32x4 a0 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + xrow + d0 + 8 * q);
                const f32x4 a1 = *reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + xrow + d0 + 8 * q + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) { tmp[e] = a0[e]; tmp[4 + e] = a1[e]; }
            } else {
                const u16x8 u = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(x) + xrow + d0 + 8 * q);
#pragma unroll
                for (int e = 0; e < 8; ++e) tmp[e] = half_to_f32<DT == kBF16 ? kBF16 : kF16>(u[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[8 * q + e] = tmp[e];
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const f32x4 cq = *reinterpret_cast<const f32x4*>(c + d0 + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e) cv[4 * q + e] = cq[e];
        }
#pragma unroll
        for (int e = 0; e < 32; ++e) dot = fmaf(xv[e], cv[e], dot);
    }
    return dot;
}

// A token row in registers, all of its loads issued together (16-bit rows kept raw).
template <int DT, int D> struct TokenRow {
    static constexpr int kVecs = DT == kF32 ? D / 4 : D / 8;  // 16-byte vectors per row
    u32x4 v[kVecs];
};

template <int DT, int D>
__device__ __forceinline__ void load_token_row(const void* x, int64_t row, TokenRow<DT, D>& r) {
    const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const char*>(x) + row * (DT == kF32 ? 4 : 2));
#pragma unroll
    for (int i = 0; i < TokenRow<DT, D>::kVecs; ++i) r.v[i] = src[i];
}

template <int DT, int D>
__device__ __forceinline__ float token_value(const TokenRow<DT, D>& r, int d) {
    if constexpr (DT == kF32) {
        return __uint_as_float(r.v[d / 4][d % 4]);
    } else {
        const uint32_t w = r.v[d / 8][(d % 8) / 2];
        return half_to_f32<DT == kBF16 ? kBF16 : kF16>(static_cast<uint16_t>(d % 2 ? w >> 16 : w & 0xffffu));
    }
}

// Canonical dot of a register-held token row with the fp32 centre row c (the same fma chain
// over d ascending as canonical_dot). The centre loads of a round (half the row for 16-bit
// tokens, a quarter for fp32 tokens, whose row takes twice the registers) are all issued
// before the chain, which keeps the assign kernel within 256 VGPRs.
template <int DT, int D>
__device__ __forceinline__ float canonical_dot_row(const TokenRow<DT, D>& r, const float* c) {
    constexpr int kRound = DT == kF32 ? D / 4 : D / 2;
    float dot = 0.0f;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += kRound) {
        f32x4 cv[kRound / 4];
#pragma unroll
        for (int i = 0; i < kRound / 4; ++i) cv[i] = reinterpret_cast<const f32x4*>(c + d0)[i];
#pragma unroll
        for (int d = 0; d < kRound; ++d) dot = fmaf(token_value<DT, D>(r, d0 + d), cv[d / 4][d % 4], dot);
    }
    return dot;
}

// Certified decision and stores for the 64 tokens of one wavefront (two 32-token column
// blocks, first token `first`): t holds each lane half's kTop smallest screened values with
// packed indices. Labels are written for valid tokens; the tile histogram (when given) counts them.
template <int DT, int D>
__device__ __forceinline__ void assign_epilogue(const KmArgs& a, const KmIter& it, int p, int b, int first, int lane,
                                                const float (&t)[2][kTop], const int (&tok)[2],
                                                const bool (&valid)[2], const float (&sq)[2], float nmax,
                                                int ibits) {
    const KmProblem& P = a.p[p];
    const int K = P.clusters;
    const int h = lane / 32;
    const uint32_t imask = (1u << ibits) - 1u;
    const float* norms = P.norms + static_cast<int64_t>(b) * K;
    const float cmax = sqrtf(nmax) * 1.001f;
    const float* cent = it.src[p] + static_cast<int64_t>(b) * K * D;
    // Index packing perturbs a value by < 2^ibits ulp.
    const float pack_rel = 1.01f * __uint_as_float((127u - 23u + static_cast<uint32_t>(ibits)) << 23);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        // The two lane halves of a token hold disjoint centres; combine their lists.
        float pt[kTop];
#pragma unroll
        for (int k = 0; k < kTop; ++k) pt[k] = __shfl_xor(t[c][k], 32, kWave);
        const float best = fminf(t[c][0], pt[0]);
        const float second = fminf(fmaxf(t[c][0], pt[0]), fminf(t[c][1], pt[1]));
        int label = static_cast<int>(__float_as_uint(best) & imask);
        // Certified decision: gap > thr (= 2E) proves `label` is the canonical argmin. E covers
        // the split-bf16 screen and the canonical fma chain (kappa), the norm inside the MFMA
        // accumulation (gamma_acc * |c|^2), fp32 rounding and the index packing.
        const float xnorm = sqrtf(sq[c]) * 1.001f;
        const float thr = 1.05f * (2.0f * a.kappa * xnorm * cmax + 2.0f * a.gamma_acc * nmax) +
                          (4.0f * 5.9604645e-8f + pack_rel) * (fabsf(best) + fabsf(second)) + 1e-30f;
        const bool flagged = valid[c] && !((second - best) > thr);
        // Every centre that can still be the canonical argmin screens within `bound`. If a
        // lane half's kTop smallest all fall inside, its list may have missed one (saturated).
        const float bound = best + thr;
        const bool saturated = flagged && (t[c][kTop - 1] <= bound || pt[kTop - 1] <= bound);
        const int64_t trow = static_cast<int64_t>(b) * P.x_stride + static_cast<int64_t>(tok[c]) * D;
        uint64_t key = ~0ull;
        if (flagged && !saturated) {
            TokenRow<DT, D> row;
            load_token_row<DT, D>(P.x, trow, row);
#pragma unroll
            for (int k = 0; k < kTop; ++k) {
                if (t[c][k] <= bound) {
                    const int j = static_cast<int>(__float_as_uint(t[c][k]) & imask);
                    const float dist = fmaf(-2.0f, canonical_dot_row<DT, D>(row, cent + static_cast<int64_t>(j) * D),
                                            norms[j]);
                    const uint64_t kj = (static_cast<uint64_t>(orderable(dist)) << 32) | static_cast<uint32_t>(j);
                    key = kj < key ? kj : key;
                }
            }
        }
        {
            const uint64_t other = __shfl_xor(key, 32, kWave);
            key = other < key ? other : key;
        }
        if (flagged && !saturated) label = static_cast<int>(key & 0xffffffffu);
        // Rare fallback: canonical re-evaluation of a saturated token over all centres, one
        // token at a time with the whole wavefront (lane i takes centres i, i + 64, ...).
        uint64_t pending = __ballot(saturated && h == 0);
        while (pending) {
            const int src = __builtin_ctzll(pending);  // lane (h == 0) holding the token
            pending &= pending - 1;
            const int64_t srow = static_cast<int64_t>(b) * P.x_stride +
                                 static_cast<int64_t>(first + 32 * c + src) * D;
            uint64_t full = ~0ull;
            TokenRow<DT, D> row;
            load_token_row<DT, D>(P.x, srow, row);
            for (int j = lane; j < K; j += kWave) {
                const float dist =
                    fmaf(-2.0f, canonical_dot_row<DT, D>(row, cent + static_cast<int64_t>(j) * D), norms[j]);
                const uint64_t kj = (static_cast<uint64_t>(orderable(dist)) << 32) | static_cast<uint32_t>(j);
                full = kj < full ? kj : full;
            }
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) {
                const uint64_t other = __shfl_xor(full, m, kWave);
                full = other < full ? other : full;
            }
            if (lane == src) label = static_cast<int>(full & 0xffffffffu);
        }
        if (valid[c] && h == 0) {
            P.labels[static_cast<int64_t>(b) * P.tokens + tok[c]] = label;
            if (it.hist[p])
                atomicAdd(it.hist[p] + (static_cast<int64_t>(b) * P.sort_tiles + tok[c] / kSortTile) * K + label, 1);
        }
    }
}

// kRaw: centre blocks are split from the fp32 centres it.src as they are loaded (the
// reference-ABI assignment, which has no buffer for the split planes).
// kDump: every screened distance (before the index is packed into it) is also written to
// it.screen, for measuring the screen's error against its certification bound.
template <int DT, int D, bool kRaw = false, bool kDump = false>
__global__ __launch_bounds__(kAssignThreads, 2) void km_assign_kernel(KmArgs a, KmIter it) {
    using T = AssignTiles<D>;
    constexpr int S = D / 16;                 // MFMA k-steps over channels
    constexpr bool kSplitX = DT != kBF16;
    __shared__ uint16_t chi[2][T::kElems];
    __shared__ uint16_t clo[2][T::kElems];
    __shared__ float cn[2][32];
    __shared__ float red[kAssignWaves];
    const int p = km_problem(a, blockIdx.x, true);
    const KmProblem& P = a.p[p];
    const int local = blockIdx.x - P.assign_begin;
    const int tiles_per_batch = static_cast<int>(ceil_div(P.tokens, kAssignTile));
    const int b = local / tiles_per_batch;
    const int tile = local % tiles_per_batch;
    const int K = P.clusters;
    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int h = lane / 32;
    const float* norms = P.norms + static_cast<int64_t>(b) * K;
    const uint16_t* hi_base = P.prep_hi + static_cast<int64_t>(b) * K * D;
    const uint16_t* lo_base = P.prep_lo + static_cast<int64_t>(b) * K * D;
    const float* raw_base = it.src[p] + static_cast<int64_t>(b) * K * D;

    CentreRegs<D> regs;
    load_centres<D, kRaw>(regs, hi_base, lo_base, raw_base, norms, 0, K, tid);
    const float n0 = norms[min(tid, K - 1)];
    float nmax = tid < K ? n0 : 0.0f;

    // x row loads are issued before any is used (a token past the end reads the last row; only
    // valid tokens' results are used): both 32-token chunks at once for bf16 input, one chunk at a time
    // when x is split (fp16/fp32), whose raw and split chunks would not fit in registers together.
    int tok[2];
    bool valid[2];
    XChunk<DT> raw[2][S];
    auto issue = [&](int c) {
        tok[c] = tile * kAssignTile + wave * 64 + 32 * c + (lane % 32);
        valid[c] = tok[c] < P.tokens;
        const int64_t xrow = static_cast<int64_t>(b) * P.x_stride + static_cast<int64_t>(min(tok[c], P.tokens - 1)) * D;
#pragma unroll
        for (int s = 0; s < S; ++s) raw[c][s] = load_x8<DT>(P.x, xrow + 16 * s + 8 * h);
    };
    if constexpr (!kSplitX) {
        issue(0);
        issue(1);
    }

    // Largest centre norm of this batch entry (for the error bound).
    for (int j = tid + blockDim.x; j < K; j += blockDim.x) nmax = fmaxf(nmax, norms[j]);
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) nmax = fmaxf(nmax, __shfl_xor(nmax, m, kWave));
    if (lane == 0) red[wave] = nmax;

    u16x8 xh[2][S], xl[2][S];
    float sq[2] = {0.0f, 0.0f};
    // Squared token norms (for the certification bound only): computed from the rows by the
    // first assign of a fit, which stores them, and read back by the later ones.
    auto split_all = [&](auto with_sq) {
        constexpr bool kSq = decltype(with_sq)::value;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            if constexpr (kSplitX) {
                tok[c] = tile * kAssignTile + wave * 64 + 32 * c + (lane % 32);
                valid[c] = tok[c] < P.tokens;
                const int64_t xrow =
                    static_cast<int64_t>(b) * P.x_stride + static_cast<int64_t>(min(tok[c], P.tokens - 1)) * D;
#pragma unroll
                for (int s = 0; s < S; ++s)
                    load_split_x8<DT, kSq>(P.x, xrow + 16 * s + 8 * h, valid[c], xh[c][s], xl[c][s], sq[c]);
            } else {
#pragma unroll
                for (int s = 0; s < S; ++s) split_x8<DT, kSq>(raw[c][s], valid[c], xh[c][s], xl[c][s], sq[c]);
            }
        }
    };
    if (it.sq_mode == 2) {
        split_all(std::false_type{});
#pragma unroll
        for (int c = 0; c < 2; ++c)
            sq[c] = P.xsq[static_cast<int64_t>(b) * P.tokens + min(tok[c], P.tokens - 1)];
    } else {
        split_all(std::true_type{});
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            sq[c] += __shfl_xor(sq[c], 32, kWave);
            if (it.sq_mode == 1 && valid[c] && h == 0) P.xsq[static_cast<int64_t>(b) * P.tokens + tok[c]] = sq[c];
        }
    }
    store_centres<D>(regs, chi[0], clo[0], cn[0], tid);
    __syncthreads();
    nmax = red[0];
#pragma unroll
    for (int w = 1; w < kAssignWaves; ++w) nmax = fmaxf(nmax, red[w]);

    // Sorted kTop smallest screened values per token and lane half (t[0] <= t[1] <= ...). The centre index
    // j is packed into the low `ibits` mantissa bits, so min/med3 track value and index
    // together; the packing error is part of the certification bound below.
    // -inf in an SGPR the compiler cannot see through: med3(t, v, -inf) = min(t, v) stays a
    // single v_med3_f32 instead of becoming a min with NaN-quieting of both operands.
    uint32_t neg_inf_bits;
    asm volatile("s_mov_b32 %0, 0xff800000" : "=s"(neg_inf_bits));
    const float neg_inf = __uint_as_float(neg_inf_bits);
    const int ibits = 32 - __builtin_clz(static_cast<unsigned>(max(K - 1, 1)));
    const uint32_t imask = (1u << ibits) - 1u;
    float t[2][kTop];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int k = 0; k < kTop; ++k) t[c][k] = kFarAway;
    const int nblocks = static_cast<int>(ceil_div(K, 32));
    // MFMA screen of the block in LDS buffer `buf`. Accumulators start at the centre norms:
    // acc = |c|^2 - 2 x.c after the chain.
    auto screen = [&](int buf, f32x16 (&acc)[2]) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 n4 = *reinterpret_cast<const f32x4*>(&cn[buf][8 * g + 4 * h]);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[c][4 * g + r] = n4[r];
            }
        const uint16_t* hrow = chi[buf] + (lane % 32) * T::kRow + 8 * h;
        const uint16_t* lrow = clo[buf] + (lane % 32) * T::kRow + 8 * h;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const bf16x8 ah = as_bf16x8(*reinterpret_cast<const u16x8*>(hrow + 16 * s));
            const bf16x8 al = as_bf16x8(*reinterpret_cast<const u16x8*>(lrow + 16 * s));
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, as_bf16x8(xh[c][s]), acc[c], 0, 0, 0);
                acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, as_bf16x8(xh[c][s]), acc[c], 0, 0, 0);
                if constexpr (kSplitX)
                    acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, as_bf16x8(xl[c][s]), acc[c], 0, 0, 0);
            }
        }
    };
    // Top-kTop tracking of block blk's screened values.
    auto track = [&](int blk, const f32x16 (&acc)[2]) {
        const int cb = blk * 32;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t j = static_cast<uint32_t>(cb + 8 * (i / 4) + 4 * h + (i % 4));
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                if constexpr (kDump) {
                    if (valid[c] && static_cast<int>(j) < K)
                        it.screen[(static_cast<int64_t>(b) * P.tokens + tok[c]) * K + j] = acc[c][i];
                }
                const float v = __uint_as_float((__float_as_uint(acc[c][i]) & ~imask) | j);
#pragma unroll
                for (int k = kTop - 1; k > 0; --k) t[c][k] = __builtin_amdgcn_fmed3f(t[c][k - 1], v, t[c][k]);
                t[c][0] = __builtin_amdgcn_fmed3f(t[c][0], v, neg_inf);
            }
        }
    };
    // Software pipeline over centre blocks: the MFMAs of block blk+1 are issued before the
    // VALU tracking of block blk, so the two overlap. Block b sits in LDS buffer b & 1; block
    // blk+2 is fetched into registers and stored into the buffer block blk has left.
    // Only called while a next block exists, so the screen and the tracking form one basic
    // block whose MFMAs and VALU instructions are interleaved explicitly (one MFMA, then a
    // share of the tracking) and execute overlapped within the wavefront.
    auto step = [&](int blk, const f32x16 (&cur)[2], f32x16 (&nxt)[2]) {
        const bool has2 = blk + 2 < nblocks;
        if (has2) load_centres<D, kRaw>(regs, hi_base, lo_base, raw_base, norms, (blk + 2) * 32, K, tid);
        screen((blk + 1) & 1, nxt);
        track(blk, cur);
        // Per channel step s its MFMAs, each followed by a share of the tracking; the centre
        // fragments of step s + kAhead are read after the first MFMA of step s, so LDS latency
        // hides behind kAhead steps of MFMAs (the norms and the first kAhead steps' fragments
        // are read up front).
        constexpr int kPerS = 2 * (kSplitX ? 3 : 2);
        constexpr int kAhead = 2;
        __builtin_amdgcn_sched_group_barrier(0x100, 4 + 2 * kAhead, 0);
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < kPerS; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (i == 0 && s + kAhead < S) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, kTrackValuPerMfma, 0);
            }
        // Uses of the candidate lists keep the tracking in this block (it would otherwise
        // be sunk past the barrier into the next block's tracking).
#pragma unroll
        for (int c = 0; c < 2; ++c) asm volatile("" ::"v"(t[c][0]), "v"(t[c][1]), "v"(t[c][2]));
        __builtin_amdgcn_sched_barrier(0);
        if (has2) store_centres<D>(regs, chi[blk & 1], clo[blk & 1], cn[blk & 1], tid);
        __syncthreads();
    };
    // With split x (fp16/fp32 input) at D = 128 the second accumulator set does not fit in
    // registers; those fits keep one set and screen, then track, each block in turn.
    constexpr bool kPipelined = !(kSplitX && D > 64);
    f32x16 acc_a[2];
    if constexpr (kPipelined) {
        f32x16 acc_b[2];
        if (nblocks > 1) load_centres<D, kRaw>(regs, hi_base, lo_base, raw_base, norms, 32, K, tid);
        screen(0, acc_a);
        if (nblocks > 1) {
            store_centres<D>(regs, chi[1], clo[1], cn[1], tid);
            __syncthreads();
        }
        int blk = 0;
        for (; blk + 2 < nblocks; blk += 2) {
            step(blk, acc_a, acc_b);
            step(blk + 1, acc_b, acc_a);
        }
        if (blk + 1 < nblocks) {
            step(blk, acc_a, acc_b);
            track(blk + 1, acc_b);
        } else {
            track(blk, acc_a);
        }
    } else {
        for (int blk = 0; blk < nblocks; ++blk) {
            const bool more = blk + 1 < nblocks;
            if (more) load_centres<D, kRaw>(regs, hi_base, lo_base, raw_base, norms, (blk + 1) * 32, K, tid);
            screen(blk & 1, acc_a);
            track(blk, acc_a);
            if (more) store_centres<D>(regs, chi[(blk + 1) & 1], clo[(blk + 1) & 1], cn[(blk + 1) & 1], tid);
            __syncthreads();
        }
    }

    assign_epilogue<DT, D>(a, it, p, b, tile * kAssignTile + wave * 64, lane, t, tok, valid, sq, nmax, ibits);
}

// PER consecutive channels of one row as fp32 (one 32-bit load for two 16-bit channels).
template <int DT, int PER>
__device__ __forceinline__ void load_pair(const void* x, int64_t e, float (&v)[PER]) {
    if constexpr (PER == 2 && DT != kF32) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(x) + e);
        v[0] = half_to_f32<DT == kBF16 ? kBF16 : kF16>(static_cast<uint16_t>(w & 0xffffu));
        v[1] = half_to_f32<DT == kBF16 ? kBF16 : kF16>(static_cast<uint16_t>(w >> 16));
    } else {
#pragma unroll
        for (int i = 0; i < PER; ++i) v[i] = load_elem<DT>(x, e + i);
    }
}

// Rows of up to N members as loaded: 16-bit inputs keep their raw 32-bit words (two
// channels per lane) until they are added, so a batch costs N registers per lane.
template <int DT, int PER, int N> struct MemberRows {
    static constexpr int W = DT == kF32 ? PER : (PER + 1) / 2;  // 32-bit words per member
    uint32_t w[N][W];
};

// Buffer resource over the rows of one batch entry of x: the member row offset goes in the
// scalar offset of each load (the member index is wave-uniform after readlane) and the lane's
// channels in the vector offset, so a load needs no per-member address registers.
struct XRows {
    __amdgpu_buffer_rsrc_t rsrc;
    int lane_bytes;  // byte offset of this lane's channels within a row
};

template <int DT, int D>
__device__ __forceinline__ XRows x_rows(const void* x, int64_t elem_offset, int tokens, int lane) {
    constexpr int E = DT == kF32 ? 4 : 2;
    constexpr int PER = D / kWave;
    const char* base = static_cast<const char*>(x) + elem_offset * E;
    const int64_t bytes = static_cast<int64_t>(tokens) * D * E;
    XRows r;
    r.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0,
                                               static_cast<int>(bytes < 0x7fffffff ? bytes : 0x7fffffff), 0x00020000);
    r.lane_bytes = lane * PER * E;
    return r;
}

// Loads the rows of cnt (1..N) members; lane u of `mine` holds the u-th member's token. The
// batch is rounded up to N loads (the extra ones re-read the last member's row) so every row
// load is in flight before the first add.
template <int DT, int PER, int N>
__device__ __forceinline__ void load_member_rows(const XRows& xr, int mine, int cnt, MemberRows<DT, PER, N>& r) {
    constexpr int D = PER * kWave;
    constexpr int E = DT == kF32 ? 4 : 2;
#pragma unroll
    for (int u = 0; u < N; ++u) {
        const int t = __builtin_amdgcn_readlane(mine, u < cnt ? u : cnt - 1);
        const int row = t * (D * E);
        if constexpr (DT == kF32 && PER == 2) {
            const auto w = __builtin_amdgcn_raw_buffer_load_b64(xr.rsrc, xr.lane_bytes, row, 0);
            r.w[u][0] = w[0];
            r.w[u][1] = w[1];
        } else if constexpr (DT == kF32 || PER == 2) {
            r.w[u][0] = __builtin_amdgcn_raw_buffer_load_b32(xr.rsrc, xr.lane_bytes, row, 0);
        } else {
            r.w[u][0] = __builtin_amdgcn_raw_buffer_load_b16(xr.rsrc, xr.lane_bytes, row, 0);
        }
    }
}

// Adds the first cnt loaded rows to s in member order.
template <int DT, int PER, int N>
__device__ __forceinline__ void fold_member_rows(const MemberRows<DT, PER, N>& r, int cnt, float (&s)[PER]) {
    constexpr int H = DT == kBF16 ? kBF16 : kF16;
#pragma unroll
    for (int u = 0; u < N; ++u)
        if (u < cnt) {
            float v[PER];
            if constexpr (DT == kF32) {
#pragma unroll
                for (int i = 0; i < PER; ++i) v[i] = __uint_as_float(r.w[u][i]);
            } else {
#pragma unroll
                for (int i = 0; i < PER; ++i) v[i] = half_to_f32<H>(static_cast<uint16_t>(r.w[u][0] >> (16 * i)));
            }
#pragma unroll
            for (int i = 0; i < PER; ++i) s[i] = s[i] + v[i];
        }
}

// Adds the rows of cnt (1..N) members to s in member order.
template <int DT, int PER, int N>
__device__ __forceinline__ void add_member_batch(const XRows& xr, int mine, int cnt, float (&s)[PER]) {
    MemberRows<DT, PER, N> r;
    load_member_rows<DT, PER, N>(xr, mine, cnt, r);
    fold_member_rows<DT, PER, N>(r, cnt, s);
}

template <int DT, int PER>
__device__ __forceinline__ void add_members(const XRows& xr, int mine, int cnt, float (&s)[PER]) {
    if (cnt > 32) add_member_batch<DT, PER, 64>(xr, mine, cnt, s);
    else if (cnt > 16) add_member_batch<DT, PER, 32>(xr, mine, cnt, s);
    else add_member_batch<DT, PER, 16>(xr, mine, cnt, s);
}

// Update of a fit, four wavefronts per workgroup. Sums member rows in original token order
// (the sorted member list is stable), divides by the count, and prepares the next
// iteration's split centres and canonical norm.
//   Wave mode (P.upd_shared == 0): each wavefront takes one cluster.
//   Shared mode: the workgroup takes one cluster (problems whose clusters average many
//   members). The member list goes 256 at a time: each wavefront loads the rows of its 64
//   consecutive members at once, then the wavefronts add their rows in turn, the running sum
//   passing through LDS, so the result is still the token-order fp32 sum while the row
//   loads of the whole 256-member stretch overlap.
constexpr int kUpdateWaves = 4;

__device__ __forceinline__ int km_update_problem(const KmArgs& a, int block) {
    int p = 0;
    while (p + 1 < a.num && !(block >= a.p[p].upd_begin && block < a.p[p].upd_begin + a.p[p].upd_blocks)) ++p;
    return p;
}

// Packing pass of the last update (cluster order): the members of one cluster, in sorted
// order m (their packed row), 16 lanes per row (8 channels each; 8 lanes at D = 64). The
// members go 64 at a time (`first`, `stride`: this wavefront's first member and step); one
// index load per lane, then the rows of 8 passes (32 or 64 rows) are requested together
// before any is used.
template <int DT> struct Raw8 {
    u32x4 v[DT == kF32 ? 2 : 1];
    __device__ __forceinline__ void load(const void* base, int64_t e) {
        const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const char*>(base) + e * (DT == kF32 ? 4 : 2));
#pragma unroll
        for (int i = 0; i < (DT == kF32 ? 2 : 1); ++i) v[i] = p[i];
    }
    __device__ __forceinline__ void store(void* base, int64_t e) const {
        u32x4* p = reinterpret_cast<u32x4*>(static_cast<char*>(base) + e * (DT == kF32 ? 4 : 2));
#pragma unroll
        for (int i = 0; i < (DT == kF32 ? 2 : 1); ++i) p[i] = v[i];
    }
    // The 8 elements as fp32 (the conversion of Row8<DT>::load).
    __device__ __forceinline__ void to_f32(float (&f)[8]) const {
        if constexpr (DT == kF32) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[i] = __uint_as_float(v[0][i]);
                f[4 + i] = __uint_as_float(v[1][i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[2 * i] = half_to_f32<DT>(static_cast<uint16_t>(v[0][i] & 0xffffu));
                f[2 * i + 1] = half_to_f32<DT>(static_cast<uint16_t>(v[0][i] >> 16));
            }
        }
    }
};

// Base-Offset payload of 8 channels of payload row `row` (codes; the row's low and scale
// from the lane holding its first channels).
__device__ __forceinline__ void store_payload(const KmProblem& P, int64_t row, int sub, int D, const uint8_t (&q)[8],
                                              float lo, float sc) {
    u32x2 packed;
    packed[0] = q[0] | (q[1] << 8) | (q[2] << 16) | (static_cast<uint32_t>(q[3]) << 24);
    packed[1] = q[4] | (q[5] << 8) | (q[6] << 16) | (static_cast<uint32_t>(q[7]) << 24);
    *reinterpret_cast<u32x2*>(P.codes + row * D + sub * 8) = packed;
    if (sub == 0) {
        P.low[row] = lo;
        P.scale[row] = sc;
    }
}

template <int DT, int D>
__device__ __forceinline__ void pack_members(const KmProblem& P, int b, int begin, int end, const float* centre,
                                             int first, int stride) {
    constexpr int G = D / 8;       // lanes per row
    constexpr int R = kWave / G;   // rows per pass
    constexpr int U = 8;           // passes in flight together
    constexpr int PASSES = kWave / R;
    const int lane = threadIdx.x % kWave;
    const int sub = lane % G, rsub = lane / G;
    const int32_t* idx = P.indices + static_cast<int64_t>(b) * P.tokens;
    const float levels = static_cast<float>((1 << P.hat_bits) - 1);
    const bool with = P.with_out != nullptr;
    float c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = centre[sub * 8 + i];
    for (int m0 = begin + first; m0 < end; m0 += stride) {
        const int cnt = min(kWave, end - m0);
        const int mine = idx[m0 + min(lane, cnt - 1)];
        for (int u0 = 0; u0 < PASSES && u0 * R < cnt; u0 += U) {
            float xv[U][8];
            Raw8<DT> wv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = min((u0 + u) * R + rsub, cnt - 1);  // clamped: every load is unconditional
                const int tok = __shfl(mine, r, kWave);
                Row8<DT>::load(P.x, b * P.x_stride + static_cast<int64_t>(tok) * D + sub * 8, xv[u]);
                if (with) wv[u].load(P.with_in, (static_cast<int64_t>(b) * P.length + tok) * D + sub * 8);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = (u0 + u) * R + rsub;
                float out[8], lo, sc;
                uint8_t q[8];
                base_offset_lane<G>(xv[u], c, levels, out, q, lo, sc);
                if (r < cnt) {
                    const int pos = m0 + r;
                    const int64_t dst = (static_cast<int64_t>(b) * P.length + pos) * D + sub * 8;
                    Row8<DT>::store(P.hat, dst, out);
                    if (with) wv[u].store(P.with_out, dst);
                    if (P.codes) store_payload(P, static_cast<int64_t>(b) * P.tokens + pos, sub, D, q, lo, sc);
                }
            }
        }
    }
}

// Text rows [tokens, length) of every problem packed in cluster order, copied into hat and
// with_out.
template <int DT, int D>
__device__ __forceinline__ void pack_text_rows(const KmArgs& a, int block) {
    constexpr int G = D / 8;
    const int sub = threadIdx.x % G;
    const int nthreads = a.text_blocks * kUpdateWaves * kWave;
    for (int p = 0; p < a.num; ++p) {
        const KmProblem& P = a.p[p];
        if (!P.hat || P.hat_order) continue;
        const int text = P.length - P.tokens;
        const int64_t rows = static_cast<int64_t>(P.batch) * text;
        for (int64_t r = (static_cast<int64_t>(block) * kUpdateWaves * kWave + threadIdx.x) / G; r < rows;
             r += nthreads / G) {
            const int64_t b = r / text;
            const int t = P.tokens + static_cast<int>(r % text);
            const int64_t dst = (b * P.length + t) * D + sub * 8;
            Row8<DT>::copy(P.x, b * P.x_stride + static_cast<int64_t>(t) * D + sub * 8, P.hat, dst);
            if (P.with_out) Row8<DT>::copy(P.with_in, dst, P.with_out, dst);
        }
    }
}

// kPack: 0 plain update; 1 the last update of a fit that packs some problem in cluster order
// (those problems' members are packed by the update itself).
template <int DT, int D, int kPack = 0>
__global__ __launch_bounds__(kUpdateWaves * kWave) void km_update_kernel(KmArgs a, KmIter it) {
    constexpr int PER = D / kWave;  // channels per lane (1 or 2)
    __shared__ float row[kUpdateWaves][D];
    __shared__ float carry[D];
    if constexpr (kPack) {
        if (static_cast<int>(blockIdx.x) >= a.total_upd_blocks) {
            pack_text_rows<DT, D>(a, blockIdx.x - a.total_upd_blocks);
            return;
        }
    }
    const int p = km_update_problem(a, blockIdx.x);
    const KmProblem& P = a.p[p];
    const int K = P.clusters;
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int local = blockIdx.x - P.upd_begin;
    const bool shared = P.upd_shared != 0;
    const int cl = shared ? local : local * kUpdateWaves + wave;  // b * K + j
    if (cl >= P.batch * K) return;  // wave mode only: the last workgroup may be partial
    const int b = cl / K;
    const int j = cl % K;
    const int32_t* off = P.offsets + static_cast<int64_t>(b) * (K + 1);
    const int begin = off[j], end = off[j + 1];
    const int32_t* idx = P.indices + static_cast<int64_t>(b) * P.tokens;
    const XRows xr = x_rows<DT, D>(P.x, static_cast<int64_t>(b) * P.x_stride, P.tokens, lane);
    float s[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) s[i] = 0.0f;
    if (!shared) {
        // Member indices arrive 64 at a time (one per lane) and are broadcast with readlane.
        for (int m0 = begin; m0 < end; m0 += kWave) {
            const int cnt = min(kWave, end - m0);
            const int mine = idx[m0 + (lane < cnt ? lane : 0)];
            add_members<DT, PER>(xr, mine, cnt, s);
        }
    } else {
        for (int base = begin; base < end; base += kUpdateWaves * kWave) {
            const int seg = base + kWave * wave;
            const int cnt = min(kWave, end - seg);  // <= 0: no members in this stretch
            MemberRows<DT, PER, kWave> rows;
            if (cnt > 0) {
                const int mine = idx[seg + min(lane, cnt - 1)];
                load_member_rows<DT, PER, kWave>(xr, mine, cnt, rows);
            }
            // Turns: wavefront w adds its rows between the workgroup's barriers w and w + 1
            // (every wavefront passes kUpdateWaves barriers per stretch).
            for (int w = 0; w < wave; ++w) __syncthreads();
            if (cnt > 0) {
                if (wave > 0 || base > begin) {
#pragma unroll
                    for (int i = 0; i < PER; ++i) s[i] = carry[lane * PER + i];
                }
                fold_member_rows<DT, PER, kWave>(rows, cnt, s);
#pragma unroll
                for (int i = 0; i < PER; ++i) carry[lane * PER + i] = s[i];
            }
            for (int w = wave; w < kUpdateWaves; ++w) __syncthreads();
        }
        if (wave != 0) {
            if constexpr (kPack) {
                if (P.hat && !P.hat_order) {
                    // The other wavefronts pack with wave 0 once it has left the centre in row[0].
                    __syncthreads();
                    pack_members<DT, D>(P, b, begin, end, row[0], kWave * wave, kWave * kUpdateWaves);
                }
            }
            return;
        }
        if (end > begin) {
#pragma unroll
            for (int i = 0; i < PER; ++i) s[i] = carry[lane * PER + i];
        }
    }
    const int count = end - begin;
    const int64_t cbase = static_cast<int64_t>(cl) * D + lane * PER;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const float mean = count > 0 ? s[i] / static_cast<float>(count) : it.src[p][cbase + i];
        it.dst[p][cbase + i] = mean;
        if (P.sums) P.sums[cbase + i] = s[i];
        row[wave][lane * PER + i] = mean;
        uint16_t hi, lo;
        split_neg2(mean, hi, lo);
        P.prep_hi[cbase + i] = hi;
        P.prep_lo[cbase + i] = lo;
    }
    // The row is read back by lane 0 of this wavefront only.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) P.norms[cl] = canonical_norm_lds(row[wave], D);
    if constexpr (kPack) {
        if (P.hat && !P.hat_order) {
            if (shared) {
                __syncthreads();  // row[0] (this wavefront's centre) is published to the others
                pack_members<DT, D>(P, b, begin, end, row[0], 0, kWave * kUpdateWaves);
            } else {
                pack_members<DT, D>(P, b, begin, end, row[wave], 0, kWave);
            }
        }
    }
}

// Packing in original order (P.hat_order 1), after the last update: row t of hat [b, length, D]
// is x's row t, Base-Offset fake-quantized (hat_bits) against the final centre of its label for
// t < tokens and copied bit for bit past it (text). G = D / 8 lanes per row (8 channels each),
// kPackRowPasses passes of 256 / G rows per workgroup over one batch entry; the labels and rows
// of every pass are requested first, then the centres the labels select.
constexpr int kPackRowPasses = 4;

template <int D> constexpr int pack_rows_per_block() { return kPackRowPasses * 256 / (D / 8); }

template <int DT, int D>
__global__ __launch_bounds__(256) void km_pack_rows_kernel(KmArgs a, KmIter it) {
    constexpr int G = D / 8;
    constexpr int R = 256 / G;
    constexpr int U = kPackRowPasses;
    int p = 0;
    while (p + 1 < a.num && !(static_cast<int>(blockIdx.x) >= a.p[p].pack_begin &&
                              static_cast<int>(blockIdx.x) < a.p[p].pack_begin + a.p[p].pack_blocks))
        ++p;
    const KmProblem& P = a.p[p];
    const int per_batch = static_cast<int>(ceil_div(P.length, R * U));
    const int local = static_cast<int>(blockIdx.x) - P.pack_begin;
    // Workgroup w runs on XCD w % kXcdCount. With a batch divisible by the XCD count (then so
    // is every pack_begin), batch entry b's rows all go to XCD b % kXcdCount, so each XCD's L2
    // fetches the centres of its own entries only.
    int b, chunk;
    if (P.batch % kXcdCount == 0) {
        const int slot = local / kXcdCount;
        b = local % kXcdCount + kXcdCount * (slot / per_batch);
        chunk = slot % per_batch;
    } else {
        b = local / per_batch;
        chunk = local % per_batch;
    }
    const int t0 = chunk * R * U + static_cast<int>(threadIdx.x) / G;
    const int sub = threadIdx.x % G;
    const int K = P.clusters;
    const float levels = static_cast<float>((1 << P.hat_bits) - 1);
    const float* cent = it.dst[p] + static_cast<int64_t>(b) * K * D + sub * 8;
    // Labels first, then the rows: the centre loads wait for the labels only, so their
    // latency overlaps the rows'.
    Raw8<DT> raw[U];
    int label[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        label[u] = P.labels[static_cast<int64_t>(b) * P.tokens + min(t0 + u * R, P.tokens - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int t = min(t0 + u * R, P.length - 1);  // clamped: every load is unconditional
        raw[u].load(P.x, static_cast<int64_t>(b) * P.x_stride + static_cast<int64_t>(t) * D + sub * 8);
    }
    float c[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int j = min(static_cast<unsigned>(label[u]), static_cast<unsigned>(K - 1));
        const f32x4* src = reinterpret_cast<const f32x4*>(cent + static_cast<int64_t>(j) * D);
        const f32x4 lo4 = src[0], hi4 = src[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[u][i] = lo4[i];
            c[u][4 + i] = hi4[i];
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int t = t0 + u * R;
        float xv[8], out[8], lo, sc;
        uint8_t q[8];
        raw[u].to_f32(xv);
        base_offset_lane<G>(xv, c[u], levels, out, q, lo, sc);
        if (t >= P.length) continue;
        const int64_t dst = (static_cast<int64_t>(b) * P.length + t) * D + sub * 8;
        if (t < P.tokens) {
            Row8<DT>::store(P.hat, dst, out);
            if (P.codes) store_payload(P, static_cast<int64_t>(b) * P.tokens + t, sub, D, q, lo, sc);
        } else {
            raw[u].store(P.hat, dst);
        }
    }
}

constexpr int kScanWaves = 8;     // clusters per update workgroup (one per wavefront)
constexpr int kScanTile = 4096;   // labels staged in LDS per step (a multiple of 256)
constexpr int kScanStep = 4 * kWave;  // labels examined per scan step (four per lane)
constexpr int kRing = 512;        // per-wave member ring (> 64 + kScanStep)

// Update without a sorted member list (peco_recompute_cluster_centers): one wavefront per
// (problem, batch, cluster), kScanWaves clusters per workgroup. The batch entry's labels stream through LDS in tiles (padded with -1 to whole steps).
// Each scan step a lane reads four consecutive labels; four ballots find the wave's members
// and their rank in token order (mbcnt over the four masks plus the lane's own earlier
// matches). Members enter a ring in token order and are summed 64 at a time, so the sum is
// the token-order fp32 sum without a sorted member list. The epilogue writes the mean
// (the previous centre when empty), count, optional sums, and the next iteration's split
// centres and canonical norm (the last two skipped when their buffers are null).
template <int DT, int D>
__global__ __launch_bounds__(kScanWaves * kWave) void km_update_scan_kernel(KmArgs a, KmIter it) {
    constexpr int PER = D / kWave;  // channels per lane (1 or 2)
    __shared__ __align__(16) int32_t lab[kScanTile];
    __shared__ int32_t ring[kScanWaves][kRing];
    __shared__ float row[kScanWaves][D];
    const int p = km_scan_problem(a, blockIdx.x);
    const KmProblem& P = a.p[p];
    const int K = P.clusters;
    const int groups = static_cast<int>(ceil_div(K, kScanWaves));
    const int local = blockIdx.x - P.scan_begin;
    const int b = local / groups;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int j = (local % groups) * kScanWaves + wave;
    const bool active = j < K;
    const int32_t* labels = P.labels + static_cast<int64_t>(b) * P.tokens;
    const XRows xr = x_rows<DT, D>(P.x, static_cast<int64_t>(b) * P.x_stride, P.tokens, lane);
    int32_t* q = ring[wave];
    float s[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) s[i] = 0.0f;
    int count = 0, head = 0, tail = 0;  // ring positions (wave-uniform, never wrapped)
    // Sums the `cnt` members at the ring head.
    auto drain = [&](int cnt) {
        // The ring writes precede this read in the wave's program order (LDS is in order).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int mine = q[(head + (lane < cnt ? lane : 0)) & (kRing - 1)];
        add_members<DT, PER>(xr, mine, cnt, s);
        __builtin_amdgcn_wave_barrier();  // ring slots are rewritten only after `mine` is read
        head += cnt;
    };
    for (int t0 = 0; t0 < P.tokens; t0 += kScanTile) {
        const int n = min(kScanTile, P.tokens - t0);
        const int padded = static_cast<int>(ceil_div(n, kScanStep)) * kScanStep;
        __syncthreads();  // the previous tile is fully scanned
        for (int i = threadIdx.x; i < padded; i += blockDim.x) lab[i] = i < n ? labels[t0 + i] : -1;
        __syncthreads();
        if (!active) continue;
        for (int c0 = 0; c0 < padded; c0 += kScanStep) {
            const int4 L = *reinterpret_cast<const int4*>(&lab[c0 + 4 * lane]);
            const bool e0 = L.x == j, e1 = L.y == j, e2 = L.z == j, e3 = L.w == j;
            const uint64_t m0 = __ballot(e0), m1 = __ballot(e1), m2 = __ballot(e2), m3 = __ballot(e3);
            if ((m0 | m1 | m2 | m3) == 0) continue;
            // Members of lower lanes (all four slots) come first, then this lane's own.
            int r = tail + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m0 >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m0), 0));
            r += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m1 >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m1), 0));
            r += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m2 >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m2), 0));
            r += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m3 >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m3), 0));
            const int tok = t0 + c0 + 4 * lane;
            if (e0) q[r & (kRing - 1)] = tok;
            r += e0;
            if (e1) q[r & (kRing - 1)] = tok + 1;
            r += e1;
            if (e2) q[r & (kRing - 1)] = tok + 2;
            r += e2;
            if (e3) q[r & (kRing - 1)] = tok + 3;
            const int add = __popcll(m0) + __popcll(m1) + __popcll(m2) + __popcll(m3);
            tail += add;
            count += add;
            while (tail - head >= kWave) drain(kWave);
        }
    }
    if (!active) return;
    if (tail > head) drain(tail - head);
    const int64_t cl = static_cast<int64_t>(b) * K + j;
    const int64_t cbase = cl * D + lane * PER;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const float mean = count > 0 ? s[i] / static_cast<float>(count) : it.src[p][cbase + i];
        it.dst[p][cbase + i] = mean;
        if (P.sums) P.sums[cbase + i] = s[i];
        row[wave][lane * PER + i] = mean;
        if (P.prep_hi) {
            uint16_t hi, lo;
            split_neg2(mean, hi, lo);
            P.prep_hi[cbase + i] = hi;
            P.prep_lo[cbase + i] = lo;
        }
    }
    if (lane == 0 && P.counts) P.counts[cl] = count;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0 && P.norms) P.norms[cl] = canonical_norm_lds(row[wave], D);
}

template <int DT, int D>
hipError_t run_fit(KmArgs& a, const KmIter* iters, int iterations, SortArgs sa, hipStream_t s) {
    hipLaunchKernelGGL((km_prep_kernel<D>), dim3(a.total_update_blocks), dim3(64), 0, s, a, iters[0]);
    for (int i = 0; i < iterations; ++i) {
        hipLaunchKernelGGL((km_assign_kernel<DT, D>), dim3(a.total_assign_blocks), dim3(kAssignThreads), 0, s, a,
                           iters[i]);
        // The sort reads the histograms this iteration's assign filled. The fused sort leaves
        // them intact and clears the other set, which the next iteration's assign fills.
        for (int q = 0; q < a.num; ++q) {
            sa.p[q].tile_hist = iters[i].hist[q];
            sa.p[q].next_hist = sa.fused ? (i % 2 == 0 ? a.p[q].tile_hist2 : a.p[q].tile_hist) : nullptr;
        }
        hipError_t e = launch_cluster_sort(sa, s, false);
        if (e != hipSuccess) return e;
        bool cluster_order = false, original = false;
        for (int q = 0; q < a.num; ++q) {
            cluster_order = cluster_order || (a.p[q].hat && !a.p[q].hat_order);
            original = original || (a.p[q].hat && a.p[q].hat_order);
        }
        if (i + 1 == iterations && cluster_order)
            hipLaunchKernelGGL((km_update_kernel<DT, D, 1>), dim3(a.total_upd_blocks + a.text_blocks),
                               dim3(kUpdateWaves * kWave), 0, s, a, iters[i]);
        else
            hipLaunchKernelGGL((km_update_kernel<DT, D>), dim3(a.total_upd_blocks), dim3(kUpdateWaves * kWave), 0, s,
                               a, iters[i]);
        if (i + 1 == iterations && original)
            hipLaunchKernelGGL((km_pack_rows_kernel<DT, D>), dim3(a.total_pack_blocks), dim3(256), 0, s, a, iters[i]);
    }
    return hipGetLastError();
}

// gamma_n = n u / (1 - n u), u = 2^-24.
double gamma_n(double n) {
    const double u = std::ldexp(1.0, -24);
    return n * u / (1.0 - n * u);
}

}  // namespace

// Coefficient of |x||c| in the bound on |screened - canonical| distance.
float km_kappa(int dtype, int dims) {
    const double split = std::ldexp(1.0, -16);
    double screen;
    if (dtype == kBF16) screen = split + gamma_n(2.0 * dims + 1) * (1.0 + std::ldexp(1.0, -7));
    else screen = 3.0 * split + gamma_n(3.0 * dims + 1) * (1.0 + std::ldexp(1.0, -6));
    const double canonical = gamma_n(dims);
    return static_cast<float>(2.0 * (screen + canonical));
}

struct KmFitDesc {
    const void* x;
    int64_t x_stride;
    const float* centers_in;
    float* centers_out;
    int32_t* labels;
    int32_t* counts;
    int32_t* indices;
    int32_t* offsets;
    int batch, tokens, clusters;
    void* hat = nullptr;             // packing by the last update (see KmProblem)
    const void* with_in = nullptr;
    void* with_out = nullptr;
    uint8_t* codes = nullptr;
    float* low = nullptr;
    float* scale = nullptr;
    int hat_bits = 0;
    int length = 0;
    int hat_order = 0;
};

// Workspace (bytes) one problem's buffers take, each rounded up to 64 bytes.
size_t km_workspace_raw(int batch, int tokens, int clusters, int dims) {
    const size_t bkd = static_cast<size_t>(batch) * clusters * dims;
    size_t bytes = 0;
    auto add = [&](size_t n) { bytes += (n + 63) / 64 * 64; };
    add(bkd * sizeof(float));                       // ping-pong centres
    add(bkd * sizeof(uint16_t));                    // prep hi
    add(bkd * sizeof(uint16_t));                    // prep lo
    add(static_cast<size_t>(batch) * clusters * sizeof(float));  // norms
    add(static_cast<size_t>(batch) * tokens * sizeof(float));    // token norms
    add(sort_workspace_ints(batch, tokens, clusters) * sizeof(int32_t));
    if (sort_fusable(tokens, clusters)) add(sort_workspace_ints(batch, tokens, clusters) * sizeof(int32_t));
    return bytes;
}

// Workspace (bytes) for one problem: its buffers plus slack for the fit's chains, whose parts
// of the buffers are rounded up separately (at most 64 bytes more per buffer and extra part).
size_t km_workspace_bytes(int batch, int tokens, int clusters, int dims) {
    return km_workspace_raw(batch, tokens, clusters, dims) + 64 * 32;
}

// A fit runs as four chains of launches, one on the caller's stream and the others on
// library-owned streams of the current device (default priority), forked from the caller's
// stream with one event and joined back to it with one event per side stream. Two layouts:
//   - by problem: each problem's batch entries (heads) in two halves, one problem per chain.
//     One problem's memory-bound launches and another's MFMA-bound ones overlap and the
//     launches' tails interleave: the 544p Q+K fit 3.46-3.47 ms, against 3.54-3.56 ms mixed;
//   - mixed, for two problems of at most kMixedTokens tokens (the 480p layer): each chain
//     takes a quarter of both problems' heads, sharing its launches (larger-K assign blocks
//     first), so the four chains carry equal work and end together: the 480p layer 1.089-1.091
//     against 1.104-1.111 ms by problem (fit 0.617-0.632 against 0.625-0.646 ms).
// More chains than the process's four hardware queues serialize (the 480p fit 0.92 ms with six
// or eight), and at 720p the layouts are within 1%. The streams and events are created once
// per device; the mutex keeps one fork-join at a time per process on the host. If the streams
// cannot be made, the problems share launches instead.
constexpr int kFitChains = 4;
constexpr int kFitParts = 2;                    // chains per problem in the by-problem layout
constexpr int kMixedTokens = 16384;
constexpr int kSideStreams = kFitChains - 1;

struct SideStream {
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};

bool side_streams(SideStream (&out)[kSideStreams], std::mutex*& m) {
    static std::mutex mutex;
    static SideStream streams[64][kSideStreams];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    std::lock_guard<std::mutex> lock(mutex);
    for (int i = 0; i < kSideStreams; ++i) {
        SideStream& s = streams[dev][i];
        if (!s.stream) {
            if (hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) != hipSuccess) return false;
            if (hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) != hipSuccess ||
                hipEventCreateWithFlags(&s.join, hipEventDisableTiming) != hipSuccess)
                return false;
        }
        out[i] = s;
    }
    m = &mutex;
    return true;
}

// Batch entries [b0, b0 + nb) of a fit description (every pointer moved to entry b0).
KmFitDesc slice_desc(const KmFitDesc& d, int b0, int nb, int dims, int dtype) {
    KmFitDesc s = d;
    const int64_t es = dtype == kF32 ? 4 : 2;
    const int64_t xs = d.x_stride > 0 ? d.x_stride : static_cast<int64_t>(d.tokens) * dims;
    const int64_t kd = static_cast<int64_t>(d.clusters) * dims;
    const int64_t rows = static_cast<int64_t>(b0) * d.length * dims;  // packed rows of entries before b0
    s.x = static_cast<const char*>(d.x) + b0 * xs * es;
    s.x_stride = xs;
    s.centers_in = d.centers_in + b0 * kd;
    s.centers_out = d.centers_out + b0 * kd;
    s.labels = d.labels + static_cast<int64_t>(b0) * d.tokens;
    s.counts = d.counts + static_cast<int64_t>(b0) * d.clusters;
    s.indices = d.indices + static_cast<int64_t>(b0) * d.tokens;
    s.offsets = d.offsets + static_cast<int64_t>(b0) * (d.clusters + 1);
    if (d.hat) s.hat = static_cast<char*>(d.hat) + rows * es;
    if (d.with_in) s.with_in = static_cast<const char*>(d.with_in) + rows * es;
    if (d.with_out) s.with_out = static_cast<char*>(d.with_out) + rows * es;
    if (d.codes) s.codes = d.codes + static_cast<int64_t>(b0) * d.tokens * dims;
    if (d.low) s.low = d.low + static_cast<int64_t>(b0) * d.tokens;
    if (d.scale) s.scale = d.scale + static_cast<int64_t>(b0) * d.tokens;
    s.batch = nb;
    return s;
}

hipError_t km_fit_launches(const KmFitDesc* descs, int num, int dims, int dtype, int iterations, void* workspace,
                           float* sums, hipStream_t stream);

// The chains of a fit (see above). By problem, the workspace holds each problem's slice of
// km_workspace_bytes in turn and the halves of a problem take their parts of it in order;
// mixed, the chains take their parts one after another. (A problem's size includes the slack
// for the extra rounding of up to kFitChains parts.)
hipError_t km_fit_chains(const KmFitDesc* descs, int num, int dims, int dtype, int iterations, void* workspace,
                         hipStream_t stream, const SideStream (&side)[kSideStreams], std::mutex& m) {
    std::lock_guard<std::mutex> lock(m);
    KmFitDesc parts[kFitChains][kMaxKm];
    int nparts[kFitChains];
    char* wsp[kFitChains];
    bool mixed = num == 2;
    for (int q = 0; q < num; ++q) mixed = mixed && descs[q].tokens <= kMixedTokens && descs[q].batch >= kFitChains;
    char* ws = static_cast<char*>(workspace);
    int home;
    if (mixed) {
        for (int c = 0; c < kFitChains; ++c) {
            wsp[c] = ws;
            nparts[c] = num;
            for (int q = 0; q < num; ++q) {
                const KmFitDesc& d = descs[q];
                const int b0 = d.batch * c / kFitChains, b1 = d.batch * (c + 1) / kFitChains;
                parts[c][q] = slice_desc(d, b0, b1 - b0, dims, dtype);
                ws += km_workspace_raw(b1 - b0, d.tokens, d.clusters, dims);
            }
        }
        home = 0;
    } else {
        int n = 0;
        for (int q = 0; q < num; ++q) {
            const KmFitDesc& d = descs[q];
            char* w = ws;
            for (int i = 0; i < kFitParts; ++i, ++n) {
                const int b0 = d.batch * i / kFitParts, b1 = d.batch * (i + 1) / kFitParts;
                parts[n][0] = slice_desc(d, b0, b1 - b0, dims, dtype);
                nparts[n] = 1;
                wsp[n] = w;
                w += km_workspace_raw(b1 - b0, d.tokens, d.clusters, dims);
            }
            ws += km_workspace_bytes(d.batch, d.tokens, d.clusters, dims);
        }
        for (int c = n; c < kFitChains; ++c) nparts[c] = 0;
        // The first half of the last problem (the larger one in the layer) on the caller's stream.
        home = (num - 1) * kFitParts;
    }
    hipError_t e = hipEventRecord(side[0].fork, stream);
    for (int i = 0; e == hipSuccess && i < kSideStreams; ++i) e = hipStreamWaitEvent(side[i].stream, side[0].fork, 0);
    int si = 0;
    for (int c = 0; e == hipSuccess && c < kFitChains; ++c) {
        if (c == home) continue;
        if (nparts[c] > 0) e = km_fit_launches(parts[c], nparts[c], dims, dtype, iterations, wsp[c], nullptr,
                                               side[si].stream);
        if (e == hipSuccess) e = hipEventRecord(side[si].join, side[si].stream);
        ++si;
    }
    if (e == hipSuccess) e = km_fit_launches(parts[home], nparts[home], dims, dtype, iterations, wsp[home], nullptr,
                                             stream);
    for (int i = 0; e == hipSuccess && i < kSideStreams; ++i) e = hipStreamWaitEvent(stream, side[i].join, 0);
    return e;
}

hipError_t km_fit(const KmFitDesc* descs, int num, int dims, int dtype, int iterations, void* workspace,
                  float* sums, hipStream_t stream) {
    bool split = !sums;  // the sums output of a one-problem fit is not sliced
    for (int q = 0; q < num; ++q) split = split && descs[q].batch >= kFitParts;
    if (split) {
        SideStream side[kSideStreams];
        std::mutex* m = nullptr;
        if (side_streams(side, m)) return km_fit_chains(descs, num, dims, dtype, iterations, workspace, stream, side, *m);
    }
    return km_fit_launches(descs, num, dims, dtype, iterations, workspace, sums, stream);
}

// One chain of launches for every problem together (the problems share each launch).
hipError_t km_fit_launches(const KmFitDesc* descs, int num, int dims, int dtype, int iterations, void* workspace,
                           float* sums, hipStream_t stream) {
    KmArgs a{};
    SortArgs sa{};
    a.num = num;
    sa.num = num;
    sa.zero_hist = 1;
    char* ws = static_cast<char*>(workspace);
    auto take = [&](size_t n) {
        char* p = ws;
        ws += (n + 63) / 64 * 64;
        return p;
    };
    int ab = 0, ub = 0;
    for (int i = 0; i < num; ++i) {
        const KmFitDesc& d = descs[i];
        KmProblem& P = a.p[i];
        const size_t bkd = static_cast<size_t>(d.batch) * d.clusters * dims;
        P.x = d.x;
        P.x_stride = d.x_stride > 0 ? d.x_stride : static_cast<int64_t>(d.tokens) * dims;
        P.centers_in = d.centers_in;
        P.centers_out = d.centers_out;
        P.centers_tmp = reinterpret_cast<float*>(take(bkd * sizeof(float)));
        P.prep_hi = reinterpret_cast<uint16_t*>(take(bkd * sizeof(uint16_t)));
        P.prep_lo = reinterpret_cast<uint16_t*>(take(bkd * sizeof(uint16_t)));
        P.norms = reinterpret_cast<float*>(take(static_cast<size_t>(d.batch) * d.clusters * sizeof(float)));
        P.xsq = reinterpret_cast<float*>(take(static_cast<size_t>(d.batch) * d.tokens * sizeof(float)));
        P.tile_hist = reinterpret_cast<int32_t*>(take(sort_workspace_ints(d.batch, d.tokens, d.clusters) * sizeof(int32_t)));
        P.tile_hist2 = sort_fusable(d.tokens, d.clusters)
                           ? reinterpret_cast<int32_t*>(take(sort_workspace_ints(d.batch, d.tokens, d.clusters) *
                                                             sizeof(int32_t)))
                           : nullptr;
        P.labels = d.labels;
        P.counts = d.counts;
        P.indices = d.indices;
        P.offsets = d.offsets;
        P.sums = (num == 1) ? sums : nullptr;
        P.batch = d.batch;
        P.tokens = d.tokens;
        P.clusters = d.clusters;
        P.sort_tiles = sort_tiles(d.tokens);
        P.assign_blocks = d.batch * static_cast<int>(ceil_div(d.tokens, kAssignTile));
        P.update_begin = ub;
        ab += P.assign_blocks;
        ub += d.batch * d.clusters;
        P.scan_blocks = d.batch * static_cast<int>(ceil_div(d.clusters, kScanWaves));
        // Clusters averaging more than one row batch (64 members) take a workgroup each.
        P.upd_shared = d.tokens > 64 * d.clusters ? 1 : 0;
        P.upd_blocks = P.upd_shared ? d.batch * d.clusters
                                    : static_cast<int>(ceil_div(static_cast<int64_t>(d.batch) * d.clusters, kUpdateWaves));
        P.hat = d.hat;
        P.with_in = d.with_in;
        P.with_out = d.with_out;
        P.codes = d.codes;
        P.low = d.low;
        P.scale = d.scale;
        P.hat_bits = d.hat_bits;
        P.length = d.length;
        P.hat_order = d.hat_order;
        if (d.hat && d.hat_order) {
            P.pack_blocks = d.batch * static_cast<int>(ceil_div(d.length, dims == 128 ? pack_rows_per_block<128>()
                                                                                     : pack_rows_per_block<64>()));
            P.pack_begin = a.total_pack_blocks;
            a.total_pack_blocks += P.pack_blocks;
        } else if (d.hat) {
            // Text copies: one 16-byte chunk per thread and row, at most 64 workgroups.
            const int64_t chunks = static_cast<int64_t>(d.batch) * std::max(d.length - d.tokens, 0) * (dims / 8);
            a.text_blocks = std::max(a.text_blocks, static_cast<int>(std::min<int64_t>(
                                                        64, std::max<int64_t>(1, ceil_div(chunks, kUpdateWaves * kWave)))));
        }
        SortProblem& q = sa.p[i];
        q.labels = d.labels;
        q.indices = d.indices;
        q.ranks = nullptr;
        q.counts = d.counts;
        q.offsets = d.offsets;
        q.tile_hist = P.tile_hist;
        q.batch = d.batch;
        q.tokens = d.tokens;
        q.clusters = d.clusters;
    }
    a.total_assign_blocks = ab;
    a.total_update_blocks = ub;
    // Longest workgroups first: assign blocks of the problem with more centres, update
    // workgroups of the problem with fewer centres (more members per cluster).
    {
        int order[kMaxKm] = {0, 1};
        if (num == 2 && a.p[1].clusters > a.p[0].clusters) std::swap(order[0], order[1]);
        int begin = 0, scan = 0, upd = 0;
        for (int i = 0; i < num; ++i) {
            a.p[order[i]].assign_begin = begin;
            begin += a.p[order[i]].assign_blocks;
            a.p[order[num - 1 - i]].scan_begin = scan;
            scan += a.p[order[num - 1 - i]].scan_blocks;
            a.p[order[num - 1 - i]].upd_begin = upd;
            upd += a.p[order[num - 1 - i]].upd_blocks;
        }
        a.total_scan_blocks = scan;
        a.total_upd_blocks = upd;
    }
    a.kappa = km_kappa(dtype, dims);
    a.gamma_acc = static_cast<float>(gamma_n(3.0 * dims + 2));
    sort_args_finalize(sa);
    // Small problems (every problem fusable) sort with one fused launch per iteration, which
    // needs the two alternating histogram sets.
    sa.fused = 1;
    for (int i = 0; i < num; ++i)
        if (!a.p[i].tile_hist2) sa.fused = 0;
    std::vector<KmIter> iters(std::max(iterations, 1));
    for (int i = 0; i < iterations; ++i) {
        for (int q = 0; q < num; ++q) {
            float* dst = ((iterations - 1 - i) % 2 == 0) ? a.p[q].centers_out : a.p[q].centers_tmp;
            iters[i].dst[q] = dst;
            iters[i].src[q] = i == 0 ? a.p[q].centers_in : iters[i - 1].dst[q];
        }
        for (int q = 0; q < num; ++q)
            iters[i].hist[q] = (sa.fused && i % 2 == 1) ? a.p[q].tile_hist2 : a.p[q].tile_hist;
        iters[i].sq_mode = i == 0 ? 1 : 2;
    }
#define PECO_FIT(DT_, D_) return run_fit<DT_, D_>(a, iters.data(), iterations, sa, stream)
    if (dims == 128) {
        if (dtype == kBF16) PECO_FIT(kBF16, 128);
        if (dtype == kF16) PECO_FIT(kF16, 128);
        if (dtype == kF32) PECO_FIT(kF32, 128);
    } else if (dims == 64) {
        if (dtype == kBF16) PECO_FIT(kBF16, 64);
        if (dtype == kF16) PECO_FIT(kF16, 64);
        if (dtype == kF32) PECO_FIT(kF32, 64);
    }
#undef PECO_FIT
    return static_cast<hipError_t>(kUnsupportedShape);
}

}  // namespace peco

using namespace peco;

namespace {
bool valid_fit(const KmFitDesc& d) {
    return d.x && d.centers_in && d.centers_out && d.labels && d.counts && d.indices && d.offsets && d.batch >= 1 &&
           d.tokens >= 1 && d.clusters >= 1 && d.clusters <= d.tokens && d.clusters <= kMaxSortClusters;
}
}  // namespace

PECO_API size_t peco_kmeans_workspace_size(int batch, int tokens, int clusters, int dims) {
    if (batch < 1 || tokens < 1 || clusters < 1 || dims < 1) return 0;
    return km_workspace_bytes(batch, tokens, clusters, dims);
}

// Fused fit of one or two independent problems (e.g. Q with KQ centres and K with KK
// centres), the second on a library stream forked from and joined to `stream`. Problem i is
// described by the i-th element of each array.
PECO_API int peco_kmeans_fit(int num_problems, const void* const* x, const int64_t* x_batch_stride,
                             const float* const* centers_in,
                             float* const* centers_out, int32_t* const* labels, int32_t* const* counts,
                             int32_t* const* sorted_indices, int32_t* const* offsets, const int* batch,
                             const int* tokens, const int* clusters, int dims, int dtype, int iterations,
                             void* workspace, size_t workspace_bytes, void* stream) {
    if (num_problems < 1 || num_problems > kMaxKm || iterations < 1 || (dims != 64 && dims != 128) ||
        (dtype != kBF16 && dtype != kF16 && dtype != kF32) || !workspace)
        return kInvalidValue;
    KmFitDesc d[kMaxKm];
    size_t need = 0;
    for (int i = 0; i < num_problems; ++i) {
        const int64_t stride = x_batch_stride ? x_batch_stride[i] : 0;
        d[i] = KmFitDesc{x[i], stride, centers_in[i], centers_out[i], labels[i], counts[i], sorted_indices[i],
                         offsets[i], batch[i], tokens[i], clusters[i]};
        if (!valid_fit(d[i]) || (stride != 0 && stride < static_cast<int64_t>(tokens[i]) * dims)) return kInvalidValue;
        need += km_workspace_bytes(batch[i], tokens[i], clusters[i], dims);
    }
    if (workspace_bytes < need) return kWorkspaceTooSmall;
    return km_fit(d, num_problems, dims, dtype, iterations, workspace, nullptr, static_cast<hipStream_t>(stream));
}

// peco_kmeans_fit whose last update also packs (fuses peco/processor.py:141-149 for the
// problems given a hat): problem i with hat[i] writes hat[i] [batch, length, dims] (rows
// [0, tokens) = x's rows Base-Offset fake-quantized with bits[i] against the final centres,
// in the final cluster order, or with hat_order 1 each at its own token position; rows
// [tokens, length) = x's rows there, so x_batch_stride[i] must cover length rows), and
// with_in[i] -> with_out[i] ([batch, length, dims], nullable, cluster order only) gathered in
// the same order with its text rows copied. codes[i], low[i] and scale[i] (nullable together;
// uint8 [batch, tokens, dims], fp32 [batch, tokens]) receive the codes, row lows and row
// scales of hat[i]'s rows [0, tokens), as peco_base_offset_encode writes them
// (peco/quantization.py:97-128), in the same order.
PECO_API int peco_kmeans_fit_pack(int num_problems, const void* const* x, const int64_t* x_batch_stride,
                                  const float* const* centers_in, float* const* centers_out, int32_t* const* labels,
                                  int32_t* const* counts, int32_t* const* sorted_indices, int32_t* const* offsets,
                                  const int* batch, const int* tokens, const int* clusters, int dims, int dtype,
                                  int iterations, void* const* hat, const int* bits, const void* const* with_in,
                                  void* const* with_out, uint8_t* const* codes, float* const* low,
                                  float* const* scale, int length, int hat_order, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    if (num_problems < 1 || num_problems > kMaxKm || iterations < 1 || (dims != 64 && dims != 128) ||
        (dtype != kBF16 && dtype != kF16 && dtype != kF32) || !workspace || !hat || !bits || !with_in || !with_out ||
        !codes || !low || !scale || (hat_order != 0 && hat_order != 1))
        return kInvalidValue;
    KmFitDesc d[kMaxKm];
    size_t need = 0;
    for (int i = 0; i < num_problems; ++i) {
        const int64_t stride = x_batch_stride ? x_batch_stride[i] : 0;
        d[i] = KmFitDesc{x[i], stride, centers_in[i], centers_out[i], labels[i], counts[i], sorted_indices[i],
                         offsets[i], batch[i], tokens[i], clusters[i]};
        if (!valid_fit(d[i]) || (stride != 0 && stride < static_cast<int64_t>(tokens[i]) * dims)) return kInvalidValue;
        if (hat[i]) {
            if ((bits[i] != 4 && bits[i] != 8) || length < tokens[i] ||
                (length > tokens[i] && stride < static_cast<int64_t>(length) * dims) || (!with_in[i] != !with_out[i]))
                return kInvalidValue;
            d[i].hat = hat[i];
            d[i].hat_bits = bits[i];
            d[i].with_in = with_in[i];
            d[i].with_out = with_out[i];
            d[i].length = length;
            d[i].hat_order = hat_order;
            if (hat_order && with_in[i]) return kInvalidValue;
            if (!codes[i] != !low[i] || !codes[i] != !scale[i]) return kInvalidValue;
            d[i].codes = codes[i];
            d[i].low = low[i];
            d[i].scale = scale[i];
        } else if (with_in[i] || with_out[i] || codes[i] || low[i] || scale[i]) {
            return kInvalidValue;
        }
        need += km_workspace_bytes(batch[i], tokens[i], clusters[i], dims);
    }
    if (workspace_bytes < need) return kWorkspaceTooSmall;
    return km_fit(d, num_problems, dims, dtype, iterations, workspace, nullptr, static_cast<hipStream_t>(stream));
}

// Reference ABI (peco/kernels/kmeans.cu:139): one assignment of fp32 x [B,N,D] to centres
// [B,C,D]. center_norms receives the canonical norms (when null, the first B*C floats of
// scratch hold them; the reference always passes both). chunk_size is accepted for ABI
// compatibility and unused. Nothing is allocated: the split-bf16 centre planes are made
// inside the assign kernel as its centre blocks are loaded.
PECO_API int peco_assign_tokens_to_centers(const float* x, const float* centers, int32_t* labels, float* scratch,
                                           float* center_norms, int batch, int tokens, int dims, int clusters,
                                           int chunk_size, void* stream) {
    (void)chunk_size;
    float* norms = center_norms ? center_norms : scratch;
    if (!x || !centers || !labels || !norms || batch < 1 || tokens < 1 || clusters < 1 ||
        (dims != 64 && dims != 128))
        return kInvalidValue;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    KmArgs a{};
    a.num = 1;
    KmProblem& P = a.p[0];
    P.x = x;
    P.x_stride = static_cast<int64_t>(tokens) * dims;
    P.prep_hi = nullptr;
    P.prep_lo = nullptr;
    P.norms = norms;
    P.labels = labels;
    P.batch = batch;
    P.tokens = tokens;
    P.clusters = clusters;
    P.sort_tiles = sort_tiles(tokens);
    a.total_assign_blocks = batch * static_cast<int>(ceil_div(tokens, kAssignTile));
    P.assign_blocks = a.total_assign_blocks;
    a.total_update_blocks = batch * clusters;
    a.kappa = km_kappa(kF32, dims);
    a.gamma_acc = static_cast<float>(gamma_n(3.0 * dims + 2));
    KmIter it{};
    it.src[0] = centers;
    if (dims == 128) {
        hipLaunchKernelGGL((km_prep_kernel<128>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        hipLaunchKernelGGL((km_assign_kernel<kF32, 128, true>), dim3(a.total_assign_blocks), dim3(kAssignThreads), 0,
                           s, a, it);
    } else {
        hipLaunchKernelGGL((km_prep_kernel<64>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        hipLaunchKernelGGL((km_assign_kernel<kF32, 64, true>), dim3(a.total_assign_blocks), dim3(kAssignThreads), 0,
                           s, a, it);
    }
    return hipGetLastError();
}

// Diagnostic: the assignment's screened distances. For bf16 x [B,N,D] and fp32 centres
// [B,C,D], screened[b,t,j] receives the value the MFMA screen of the assign kernel compares
// (|c_j|^2 - 2 x_t.c_j from split-bf16 centres); center_norms receives the canonical norms and
// labels the certified labels. Used to measure the screen error against its bound.
PECO_API int peco_kmeans_screen(const void* x, int dtype, const float* centers, float* center_norms,
                                int32_t* labels, float* screened, int batch, int tokens, int dims, int clusters,
                                void* stream) {
    if (!x || !centers || !center_norms || !labels || !screened || batch < 1 || tokens < 1 || clusters < 1 ||
        (dims != 64 && dims != 128))
        return kInvalidValue;
    if (dtype != kBF16) return kUnsupportedDtype;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    KmArgs a{};
    a.num = 1;
    KmProblem& P = a.p[0];
    P.x = x;
    P.x_stride = static_cast<int64_t>(tokens) * dims;
    P.norms = center_norms;
    P.labels = labels;
    P.batch = batch;
    P.tokens = tokens;
    P.clusters = clusters;
    P.sort_tiles = sort_tiles(tokens);
    a.total_assign_blocks = batch * static_cast<int>(ceil_div(tokens, kAssignTile));
    P.assign_blocks = a.total_assign_blocks;
    a.total_update_blocks = batch * clusters;
    a.kappa = km_kappa(kBF16, dims);
    a.gamma_acc = static_cast<float>(gamma_n(3.0 * dims + 2));
    KmIter it{};
    it.src[0] = centers;
    it.screen = screened;
    if (dims == 128) {
        hipLaunchKernelGGL((km_prep_kernel<128>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        hipLaunchKernelGGL((km_assign_kernel<kBF16, 128, true, true>), dim3(a.total_assign_blocks),
                           dim3(kAssignThreads), 0, s, a, it);
    } else {
        hipLaunchKernelGGL((km_prep_kernel<64>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        hipLaunchKernelGGL((km_assign_kernel<kBF16, 64, true, true>), dim3(a.total_assign_blocks),
                           dim3(kAssignThreads), 0, s, a, it);
    }
    return hipGetLastError();
}

// Screen error bound coefficients of the assignment for bf16 tokens: kappa (of |x||c|) and
// gamma (of |c|^2), as the certified decision uses them.
PECO_API void peco_kmeans_screen_bound(int dims, float* kappa, float* gamma) {
    if (kappa) *kappa = km_kappa(kBF16, dims);
    if (gamma) *gamma = static_cast<float>(gamma_n(3.0 * dims + 2));
}

// Reference ABI (peco/kernels/kmeans.cu:179): means/counts of fp32 x [B,N,D] for labels
// [B,N]; sums receives the per-cluster sums; empty clusters keep `previous`.
PECO_API int peco_recompute_cluster_centers(const float* x, const int32_t* labels, const float* previous, float* sums,
                                            int32_t* counts, float* means, int batch, int tokens, int dims,
                                            int clusters, void* stream) {
    if (!x || !labels || !previous || !counts || !means || batch < 1 || tokens < 1 || clusters < 1 ||
        (dims != 64 && dims != 128))
        return kInvalidValue;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // Members are found from the labels directly (labels outside [0, clusters) join no
    // cluster); no sort, no workspace.
    KmArgs a{};
    a.num = 1;
    KmProblem& P = a.p[0];
    P.x = x;
    P.x_stride = static_cast<int64_t>(tokens) * dims;
    P.labels = const_cast<int32_t*>(labels);
    P.counts = counts;
    P.sums = sums;
    P.batch = batch;
    P.tokens = tokens;
    P.clusters = clusters;
    P.scan_begin = 0;
    P.scan_blocks = batch * static_cast<int>(ceil_div(clusters, kScanWaves));
    a.total_scan_blocks = P.scan_blocks;
    KmIter it{};
    it.src[0] = previous;
    it.dst[0] = means;
    if (dims == 128)
        hipLaunchKernelGGL((km_update_scan_kernel<kF32, 128>), dim3(a.total_scan_blocks), dim3(kScanWaves * kWave), 0,
                           s, a, it);
    else
        hipLaunchKernelGGL((km_update_scan_kernel<kF32, 64>), dim3(a.total_scan_blocks), dim3(kScanWaves * kWave), 0,
                           s, a, it);
    return hipGetLastError();
}
