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
// its four smallest screened values with the centre index packed into the low mantissa
// bits. With best and second best b1 <= b2 and the bound E, b2 - b1 > 2E proves that the
// centre of b1 is the canonical argmin. Otherwise every centre screening within b1 + 2E is
// a candidate (all of them are among the kept four unless that list is saturated); the
// candidates get the canonical fp32 distance in-kernel, lowest index on ties, and a
// saturated list falls back to evaluating all centres. Labels are therefore identical to the
// canonical fixed-order fp32 definition, not approximately equal.
//
// Per iteration: assign (+ per-tile label histogram via global atomics) -> sort scan ->
// sort place (stable counting sort, also yields the final permutation for stage 3) ->
// update (sequential per-cluster sums in token order; also prepares the next iteration's
// split-bf16 centres and canonical norms). Q and K fits share every launch.
#include "common.hpp"
#include "sort.hpp"

#include <algorithm>
#include <cmath>
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
    int32_t* tile_hist;     // [batch, sort tiles, K]
    float* sums;            // nullable [batch, K, D]: per-cluster sums of the last update
    int batch, tokens, clusters;
    int assign_begin;       // first linear assign block (batch * ceil(tokens/256) blocks)
    int update_begin;       // first linear update block (batch * K blocks)
    int sort_tiles;
};

constexpr int kMaxKm = 2;
constexpr int kAssignTile = 256;  // tokens per assign workgroup (4 waves x 64 tokens)

struct KmArgs {
    KmProblem p[kMaxKm];
    int num;
    int total_assign_blocks;
    int total_update_blocks;
    float kappa;      // bound coefficient: |screened - canonical| <= kappa*|x||c| + rounding terms
    float gamma_acc;  // gamma of the MFMA accumulation length (applied to the norm term)
};

struct KmIter {
    const float* src[kMaxKm];  // centres used by this iteration
    float* dst[kMaxKm];        // means written by this iteration
};

namespace {

__device__ __forceinline__ int km_problem(const KmArgs& a, int block, bool assign) {
    int p = 0;
    if (assign) {
        while (p + 1 < a.num && block >= a.p[p + 1].assign_begin) ++p;
    } else {
        while (p + 1 < a.num && block >= a.p[p + 1].update_begin) ++p;
    }
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

// Initial preparation: norms + split of the initial centres; clears the tile histograms.
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
        uint16_t hi, lo;
        split_neg2(v, hi, lo);
        P.prep_hi[static_cast<int64_t>(local) * D + d] = hi;
        P.prep_lo[static_cast<int64_t>(local) * D + d] = lo;
    }
    __syncthreads();
    if (threadIdx.x == 0) P.norms[local] = canonical_norm_lds(row, D);
    // Clear this problem's tile histograms (strided over the problem's blocks).
    const int64_t hist = static_cast<int64_t>(P.batch) * P.sort_tiles * P.clusters;
    const int64_t nblocks = static_cast<int64_t>(P.batch) * P.clusters;
    for (int64_t i = static_cast<int64_t>(local) * kWave + threadIdx.x; i < hist; i += nblocks * kWave)
        P.tile_hist[i] = 0;
}

// x operand (B of the MFMA): 8 consecutive channels of one token as bf16 (hi, and lo when split).
template <int DT>
__device__ __forceinline__ void load_x8(const void* x, int64_t e, bool valid, u16x8& hi, u16x8& lo, float& sq) {
    if (!valid) {
        hi = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        lo = hi;
        return;
    }
    if constexpr (DT == kBF16) {
        hi = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(x) + e);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float f = bf16_bits_to_f32(hi[i]);
            sq = fmaf(f, f, sq);
        }
    } else {
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
            sq = fmaf(f[i], f[i], sq);
        }
    }
}

// Assign: one workgroup = 256 tokens of one (problem, batch); wave w owns tokens
// [64w, 64w+64) as two 32-token MFMA column blocks. Centres stream through LDS in blocks of
// 32 (split-bf16 hi/lo rows + canonical norms), double-buffered with a register prefetch.
// MFMA 32x32x16: A = centres (32 rows x 16 channels), B = tokens (16 channels x 32 tokens);
// lane l holds token l%32 of each column block and centres 8*(i/4)+4*(l/32)+i%4.
// Screened distance of centres past K (finite, so index bits can be packed into it).
constexpr float kFarAway = 1.0e37f;

template <int D> struct AssignTiles {
    static constexpr int kRow = D + 8;                 // padded LDS row (16-bit elements)
    static constexpr int kElems = 32 * kRow;
    static constexpr int kChunks = D / 8;              // 16-byte chunks per row
    static constexpr int kLoads = 32 * kChunks / 256;  // 16-byte loads per thread per array
};

template <int D> struct CentreRegs {
    u32x4 hi[AssignTiles<D>::kLoads], lo[AssignTiles<D>::kLoads];
    float norm;
};

template <int D>
__device__ __forceinline__ void load_centres(CentreRegs<D>& R, const uint16_t* hi_base, const uint16_t* lo_base,
                                             const float* norms, int cb, int K, int tid) {
    using T = AssignTiles<D>;
#pragma unroll
    for (int i = 0; i < T::kLoads; ++i) {
        const int id = i * 256 + tid;
        const int row = min(cb + id / T::kChunks, K - 1);  // rows past K are never selected
        const int64_t e = static_cast<int64_t>(row) * D + (id % T::kChunks) * 8;
        R.hi[i] = *reinterpret_cast<const u32x4*>(hi_base + e);
        R.lo[i] = *reinterpret_cast<const u32x4*>(lo_base + e);
    }
    if (tid < 32) R.norm = cb + tid < K ? norms[cb + tid] : kFarAway;
}

template <int D>
__device__ __forceinline__ void store_centres(const CentreRegs<D>& R, uint16_t* hi, uint16_t* lo, float* nrm, int tid) {
    using T = AssignTiles<D>;
#pragma unroll
    for (int i = 0; i < T::kLoads; ++i) {
        const int id = i * 256 + tid;
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

template <int DT, int D>
__global__ __launch_bounds__(256, 2) void km_assign_kernel(KmArgs a, KmIter it) {
    using T = AssignTiles<D>;
    constexpr int S = D / 16;                 // MFMA k-steps over channels
    constexpr bool kSplitX = DT != kBF16;
    __shared__ uint16_t chi[2][T::kElems];
    __shared__ uint16_t clo[2][T::kElems];
    __shared__ float cn[2][32];
    __shared__ float red[4];
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

    CentreRegs<D> regs;
    load_centres<D>(regs, hi_base, lo_base, norms, 0, K, tid);

    // Largest centre norm of this batch entry (for the error bound).
    float nmax = 0.0f;
    for (int j = tid; j < K; j += blockDim.x) nmax = fmaxf(nmax, norms[j]);
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) nmax = fmaxf(nmax, __shfl_xor(nmax, m, kWave));
    if (lane == 0) red[wave] = nmax;

    int tok[2];
    bool valid[2];
    u16x8 xh[2][S], xl[2][S];
    float sq[2] = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        tok[c] = tile * kAssignTile + wave * 64 + 32 * c + (lane % 32);
        valid[c] = tok[c] < P.tokens;
        const int64_t xrow = static_cast<int64_t>(b) * P.x_stride + static_cast<int64_t>(tok[c]) * D;
#pragma unroll
        for (int s = 0; s < S; ++s) load_x8<DT>(P.x, xrow + 16 * s + 8 * h, valid[c], xh[c][s], xl[c][s], sq[c]);
        sq[c] += __shfl_xor(sq[c], 32, kWave);
    }
    store_centres<D>(regs, chi[0], clo[0], cn[0], tid);
    __syncthreads();
    nmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));

    // Sorted four smallest screened values per token (t[0] <= ... <= t[3]). The centre index
    // j is packed into the low `ibits` mantissa bits, so min/med3 track value and index
    // together; the packing error is part of the certification bound below.
    const int ibits = 32 - __builtin_clz(static_cast<unsigned>(max(K - 1, 1)));
    const uint32_t imask = (1u << ibits) - 1u;
    float t[2][4];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) t[c][k] = kFarAway;
    const int nblocks = static_cast<int>(ceil_div(K, 32));
    for (int blk = 0; blk < nblocks; ++blk) {
        const int buf = blk & 1;
        const bool more = blk + 1 < nblocks;
        if (more) load_centres<D>(regs, hi_base, lo_base, norms, (blk + 1) * 32, K, tid);
        // Accumulators start at the centre norms: acc = |c|^2 - 2 x.c after the chain.
        f32x16 acc[2];
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
        const int cb = blk * 32;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t j = static_cast<uint32_t>(cb + 8 * (i / 4) + 4 * h + (i % 4));
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const float v = __uint_as_float((__float_as_uint(acc[c][i]) & ~imask) | j);
                t[c][3] = __builtin_amdgcn_fmed3f(t[c][2], v, t[c][3]);
                t[c][2] = __builtin_amdgcn_fmed3f(t[c][1], v, t[c][2]);
                t[c][1] = __builtin_amdgcn_fmed3f(t[c][0], v, t[c][1]);
                t[c][0] = fminf(t[c][0], v);
            }
        }
        if (more) store_centres<D>(regs, chi[buf ^ 1], clo[buf ^ 1], cn[buf ^ 1], tid);
        __syncthreads();
    }

    const float cmax = sqrtf(nmax) * 1.001f;
    const float* cent = it.src[p] + static_cast<int64_t>(b) * K * D;
    // Index packing perturbs a value by < 2^ibits ulp.
    const float pack_rel = 1.01f * __uint_as_float((127u - 23u + static_cast<uint32_t>(ibits)) << 23);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        // The two lane halves of a token hold disjoint centres; combine their lists.
        float pt[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) pt[k] = __shfl_xor(t[c][k], 32, kWave);
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
        // lane's four smallest all fall inside, its list may have missed one (saturated).
        const float bound = best + thr;
        const bool saturated = flagged && (t[c][3] <= bound || pt[3] <= bound);
        const int64_t trow = static_cast<int64_t>(b) * P.x_stride + static_cast<int64_t>(tok[c]) * D;
        uint64_t key = ~0ull;
        if (flagged && !saturated) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (t[c][k] <= bound) {
                    const int j = static_cast<int>(__float_as_uint(t[c][k]) & imask);
                    const float dist = fmaf(-2.0f, canonical_dot<DT, D>(P.x, trow, cent + static_cast<int64_t>(j) * D),
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
                                 static_cast<int64_t>(tile * kAssignTile + wave * 64 + 32 * c + src) * D;
            uint64_t full = ~0ull;
            for (int j = lane; j < K; j += kWave) {
                const float dist =
                    fmaf(-2.0f, canonical_dot<DT, D>(P.x, srow, cent + static_cast<int64_t>(j) * D), norms[j]);
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
            atomicAdd(P.tile_hist + (static_cast<int64_t>(b) * P.sort_tiles + tok[c] / kSortTile) * K + label, 1);
        }
    }
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

// Update: one wavefront per (problem, batch, cluster). Sums member rows in original token
// order (the sorted member list is stable), divides by the count, and prepares the next
// iteration's split centres and canonical norm.
template <int DT, int D>
__global__ __launch_bounds__(64) void km_update_kernel(KmArgs a, KmIter it) {
    constexpr int PER = D / kWave;  // channels per lane (1 or 2)
    __shared__ float row[D];
    const int p = km_problem(a, blockIdx.x, false);
    const KmProblem& P = a.p[p];
    const int local = blockIdx.x - P.update_begin;  // b * K + j
    const int K = P.clusters;
    const int b = local / K;
    const int j = local % K;
    const int lane = threadIdx.x;
    const int32_t* off = P.offsets + static_cast<int64_t>(b) * (K + 1);
    const int begin = off[j], end = off[j + 1];
    const int32_t* idx = P.indices + static_cast<int64_t>(b) * P.tokens;
    const int64_t xbase = static_cast<int64_t>(b) * P.x_stride + lane * PER;
    float s[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) s[i] = 0.0f;
    // Member indices arrive 64 at a time (one per lane) and are broadcast with readlane; all
    // of a chunk's row loads (32 bits per lane) are in flight before the adds, which stay in
    // member (= token) order.
    for (int m0 = begin; m0 < end; m0 += kWave) {
        const int cnt = min(kWave, end - m0);
        const int mine = lane < cnt ? idx[m0 + lane] : idx[m0];
        if (cnt == kWave) {
            float v[kWave][PER];
#pragma unroll
            for (int u = 0; u < kWave; ++u) {
                const int t = __builtin_amdgcn_readlane(mine, u);
                load_pair<DT, PER>(P.x, xbase + static_cast<int64_t>(t) * D, v[u]);
            }
#pragma unroll
            for (int u = 0; u < kWave; ++u)
#pragma unroll
                for (int i = 0; i < PER; ++i) s[i] = s[i] + v[u][i];
        } else {
            int j = 0;
            for (; j + 16 <= cnt; j += 16) {
                float v[16][PER];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int t = __builtin_amdgcn_readlane(mine, j + u);
                    load_pair<DT, PER>(P.x, xbase + static_cast<int64_t>(t) * D, v[u]);
                }
#pragma unroll
                for (int u = 0; u < 16; ++u)
#pragma unroll
                    for (int i = 0; i < PER; ++i) s[i] = s[i] + v[u][i];
            }
            for (; j < cnt; ++j) {
                const int t = __builtin_amdgcn_readlane(mine, j);
                float v[PER];
                load_pair<DT, PER>(P.x, xbase + static_cast<int64_t>(t) * D, v);
#pragma unroll
                for (int i = 0; i < PER; ++i) s[i] = s[i] + v[i];
            }
        }
    }
    const int count = end - begin;
    const int64_t cbase = static_cast<int64_t>(local) * D + lane * PER;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const float mean = count > 0 ? s[i] / static_cast<float>(count) : it.src[p][cbase + i];
        it.dst[p][cbase + i] = mean;
        if (P.sums) P.sums[cbase + i] = s[i];
        row[lane * PER + i] = mean;
        uint16_t hi, lo;
        split_neg2(mean, hi, lo);
        P.prep_hi[cbase + i] = hi;
        P.prep_lo[cbase + i] = lo;
    }
    __syncthreads();
    if (lane == 0) P.norms[local] = canonical_norm_lds(row, D);
}

template <int DT, int D>
hipError_t run_fit(KmArgs& a, const KmIter* iters, int iterations, const SortArgs& sa, hipStream_t s) {
    hipLaunchKernelGGL((km_prep_kernel<D>), dim3(a.total_update_blocks), dim3(64), 0, s, a, iters[0]);
    for (int i = 0; i < iterations; ++i) {
        hipLaunchKernelGGL((km_assign_kernel<DT, D>), dim3(a.total_assign_blocks), dim3(256), 0, s, a, iters[i]);
        hipError_t e = launch_cluster_sort(sa, s, false);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((km_update_kernel<DT, D>), dim3(a.total_update_blocks), dim3(64), 0, s, a, iters[i]);
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
};

// Workspace (bytes) for one problem.
size_t km_workspace_bytes(int batch, int tokens, int clusters, int dims) {
    const size_t bkd = static_cast<size_t>(batch) * clusters * dims;
    size_t bytes = 0;
    auto add = [&](size_t n) { bytes += (n + 63) / 64 * 64; };
    add(bkd * sizeof(float));                       // ping-pong centres
    add(bkd * sizeof(uint16_t));                    // prep hi
    add(bkd * sizeof(uint16_t));                    // prep lo
    add(static_cast<size_t>(batch) * clusters * sizeof(float));  // norms
    add(sort_workspace_ints(batch, tokens, clusters) * sizeof(int32_t));
    return bytes;
}

hipError_t km_fit(const KmFitDesc* descs, int num, int dims, int dtype, int iterations, void* workspace,
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
        P.tile_hist = reinterpret_cast<int32_t*>(take(sort_workspace_ints(d.batch, d.tokens, d.clusters) * sizeof(int32_t)));
        P.labels = d.labels;
        P.counts = d.counts;
        P.indices = d.indices;
        P.offsets = d.offsets;
        P.sums = (num == 1) ? sums : nullptr;
        P.batch = d.batch;
        P.tokens = d.tokens;
        P.clusters = d.clusters;
        P.sort_tiles = sort_tiles(d.tokens);
        P.assign_begin = ab;
        P.update_begin = ub;
        ab += d.batch * static_cast<int>(ceil_div(d.tokens, kAssignTile));
        ub += d.batch * d.clusters;
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
    a.kappa = km_kappa(dtype, dims);
    a.gamma_acc = static_cast<float>(gamma_n(3.0 * dims + 2));
    sort_args_finalize(sa);
    std::vector<KmIter> iters(std::max(iterations, 1));
    for (int i = 0; i < iterations; ++i) {
        for (int q = 0; q < num; ++q) {
            float* dst = ((iterations - 1 - i) % 2 == 0) ? a.p[q].centers_out : a.p[q].centers_tmp;
            iters[i].dst[q] = dst;
            iters[i].src[q] = i == 0 ? a.p[q].centers_in : iters[i - 1].dst[q];
        }
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
// centres) sharing every launch. Problem i is described by the i-th element of each array.
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

// Reference ABI (peco/kernels/kmeans.cu:139): one assignment of fp32 x [B,N,D] to centres
// [B,C,D]. scratch/chunk_size are accepted for ABI compatibility and unused; center_norms
// receives the canonical norms. Internal buffers come from the stream-ordered allocator.
PECO_API int peco_assign_tokens_to_centers(const float* x, const float* centers, int32_t* labels, float* scratch,
                                           float* center_norms, int batch, int tokens, int dims, int clusters,
                                           int chunk_size, void* stream) {
    (void)scratch;
    (void)chunk_size;
    if (!x || !centers || !labels || batch < 1 || tokens < 1 || clusters < 1 || (dims != 64 && dims != 128))
        return kInvalidValue;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    KmArgs a{};
    a.num = 1;
    KmProblem& P = a.p[0];
    const size_t bkd = static_cast<size_t>(batch) * clusters * dims;
    const size_t hist = sort_workspace_ints(batch, tokens, clusters);
    void* buf = nullptr;
    const size_t bytes = bkd * 4 + (center_norms ? 0 : static_cast<size_t>(batch) * clusters * 4) + hist * 4 + 256;
    hipError_t e = hipMallocAsync(&buf, bytes, s);
    if (e != hipSuccess) return e;
    char* w = static_cast<char*>(buf);
    P.x = x;
    P.x_stride = static_cast<int64_t>(tokens) * dims;
    P.prep_hi = reinterpret_cast<uint16_t*>(w);
    P.prep_lo = P.prep_hi + bkd;
    w += bkd * 4;
    if (center_norms) P.norms = center_norms;
    else { P.norms = reinterpret_cast<float*>(w); w += static_cast<size_t>(batch) * clusters * 4; }
    P.tile_hist = reinterpret_cast<int32_t*>(w);
    P.labels = labels;
    P.batch = batch;
    P.tokens = tokens;
    P.clusters = clusters;
    P.sort_tiles = sort_tiles(tokens);
    a.total_assign_blocks = batch * static_cast<int>(ceil_div(tokens, kAssignTile));
    a.total_update_blocks = batch * clusters;
    a.kappa = km_kappa(kF32, dims);
    a.gamma_acc = static_cast<float>(gamma_n(3.0 * dims + 2));
    KmIter it{};
    it.src[0] = centers;
    if (dims == 128) {
        hipLaunchKernelGGL((km_prep_kernel<128>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        hipLaunchKernelGGL((km_assign_kernel<kF32, 128>), dim3(a.total_assign_blocks), dim3(256), 0, s, a, it);
    } else {
        hipLaunchKernelGGL((km_prep_kernel<64>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        hipLaunchKernelGGL((km_assign_kernel<kF32, 64>), dim3(a.total_assign_blocks), dim3(256), 0, s, a, it);
    }
    e = hipGetLastError();
    hipError_t f = hipFreeAsync(buf, s);
    return e != hipSuccess ? e : f;
}

// Reference ABI (peco/kernels/kmeans.cu:179): means/counts of fp32 x [B,N,D] for labels
// [B,N]; sums receives the per-cluster sums; empty clusters keep `previous`.
PECO_API int peco_recompute_cluster_centers(const float* x, const int32_t* labels, const float* previous, float* sums,
                                            int32_t* counts, float* means, int batch, int tokens, int dims,
                                            int clusters, void* stream) {
    if (!x || !labels || !previous || !counts || !means || batch < 1 || tokens < 1 || clusters < 1 ||
        clusters > kMaxSortClusters || (dims != 64 && dims != 128))
        return kInvalidValue;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t bkd = static_cast<size_t>(batch) * clusters * dims;
    const size_t hist = sort_workspace_ints(batch, tokens, clusters);
    const size_t idx = static_cast<size_t>(batch) * tokens;
    const size_t off = static_cast<size_t>(batch) * (clusters + 1);
    const size_t nrm = static_cast<size_t>(batch) * clusters;
    void* buf = nullptr;
    hipError_t e = hipMallocAsync(&buf, (bkd * 2 + hist + idx + off + nrm) * 4 + 256, s);
    if (e != hipSuccess) return e;
    char* w = static_cast<char*>(buf);
    SortArgs sa{};
    sa.num = 1;
    SortProblem& q = sa.p[0];
    q.labels = labels;
    q.indices = reinterpret_cast<int32_t*>(w);
    w += idx * 4;
    q.offsets = reinterpret_cast<int32_t*>(w);
    w += off * 4;
    q.tile_hist = reinterpret_cast<int32_t*>(w);
    w += hist * 4;
    q.counts = counts;
    q.ranks = nullptr;
    q.batch = batch;
    q.tokens = tokens;
    q.clusters = clusters;
    sort_args_finalize(sa);
    e = launch_cluster_sort(sa, s, true);
    if (e == hipSuccess) {
        KmArgs a{};
        a.num = 1;
        KmProblem& P = a.p[0];
        P.x = x;
        P.x_stride = static_cast<int64_t>(tokens) * dims;
        P.indices = q.indices;
        P.offsets = q.offsets;
        P.prep_hi = reinterpret_cast<uint16_t*>(w);
        P.prep_lo = P.prep_hi + bkd;
        w += bkd * 4;
        P.norms = reinterpret_cast<float*>(w);
        P.sums = sums;
        P.batch = batch;
        P.tokens = tokens;
        P.clusters = clusters;
        a.total_update_blocks = batch * clusters;
        KmIter it{};
        it.src[0] = previous;
        it.dst[0] = means;
        if (dims == 128)
            hipLaunchKernelGGL((km_update_kernel<kF32, 128>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        else
            hipLaunchKernelGGL((km_update_kernel<kF32, 64>), dim3(a.total_update_blocks), dim3(64), 0, s, a, it);
        e = hipGetLastError();
    }
    hipError_t f = hipFreeAsync(buf, s);
    return e != hipSuccess ? e : f;
}
