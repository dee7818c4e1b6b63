// Cluster-pair selection (peco/clustering.py:140-186) and the text partition
// (peco/processor.py:68-84) in one launch.
//
// One wavefront per (batch*head, query cluster) row:
//   score_j = (Cq . Ck_j) * fl(D^-0.5)                (fma chain over d ascending)
//   logit_j = score_j + log(count_j), or -inf for an empty key cluster
//   prob_j  = exp(logit_j - rowmax) / max(sum, FLT_MIN) (rowmax = 0 when no key is non-empty)
//   order   = probabilities descending, ties by ascending index (torch's stable sort)
//   keep_k  = (cumsum_k - prob_k) < p over that order, cumsum accumulated in double and
//             rounded per element (torch's CPU cumsum); p == 1 keeps all; the first
//             max(1, minimum) entries are always kept
//   map[c, j] = keep && count_j > 0 && qcount_c > 0
// With `extend`, the map gains the valid-text and padding groups: the valid-text row and
// column pair with everything but padding, padding pairs only with itself, and the size
// vectors gain (valid_text, text - valid_text).
//
// Layout: a workgroup of kSelWaves waves owns kSelWaves query rows of one batch entry and
// streams the key centroids through LDS in blocks of 64 rows (row stride dims+1 floats, so
// lane j reading row j is bank-conflict free), with up to four blocks in flight in registers
// (at 480p 10% faster than one); lane j of a wave scores key j of the block.
// Each wave then holds its row's ck keys in registers, KPL = ck_pow2/64 per lane, and sorts
// them with a register bitonic network (cross-lane stages by xor shuffles).
//
// The kept set is a prefix of the sorted order: with probabilities descending and the
// running sum nondecreasing, cum_{k+1} - prob_{k+1} >= cum_k - prob_k exactly, so the
// rounded `before` values are nondecreasing too. The sequential double walk therefore
// stops at the first entry past the minimum whose `before` reaches p.
#include "common.hpp"
#include "work.hpp"

#include <algorithm>
#include <cmath>

namespace peco {
namespace {

constexpr int kSelWaves = 8;
constexpr int kSelThreads = kSelWaves * kWave;
constexpr int kSelBlock = 64;
constexpr int kSelMaxDims = 256;
// Staged floats per thread and key block: kWide (dims up to kSelMaxDims) or not (up to 128).
template <bool kWide> constexpr int sel_loads() { return kSelBlock * (kWide ? kSelMaxDims : 128) / kSelThreads; }
// Key blocks in flight: 64 staged floats per thread (32 when each lane also holds 16 or more
// keys, whose registers the row needs), at most the blocks there are.
template <int KPL, bool kWide> constexpr int sel_depth() {
    const int d = (KPL >= 16 ? 32 : 64) / sel_loads<kWide>();
    return d < 1 ? 1 : (d > KPL ? KPL : d);
}
constexpr int kSelBatch = 32;

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const int lo = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v)), mask, kWave);
    const int hi = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v >> 32)), mask, kWave);
    return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// Inverse of the key's high word (~orderable(prob)).
__device__ __forceinline__ float key_prob(uint32_t high) {
    const uint32_t ord = ~high;
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}

// Kept-segment list of one map row, written by one wavefront: lane l takes clusters l,
// l + 64, ... of the extended cluster order, whose rows are [min(sk, prefix), min(sk, prefix +
// size)) of the key stream. A kept cluster with rows extends the current segment when the
// previous cluster with rows was kept too (their rows are adjacent), else it opens one.
// Returns the row's stream length L.
// kcnt[i] holds the size of key cluster 64 i + lane (0 past ck).
template <int KPL, typename Kept>
__device__ int write_segments(int2* __restrict__ srow, const int (&kcnt)[KPL], int ck, int ce, int valid_text,
                              int text, int sk, Kept kept) {
    const int lane = lane_id();
    const uint64_t below = (1ull << lane) - 1ull;
    int pre = 0, run = 0, nseg = 0;
    bool prev_on = false;
#pragma unroll
    for (int ch = 0; ch <= KPL; ++ch) {
        const int j0 = ch * kWave;
        if (j0 >= ce) break;
        const int j = j0 + lane;
        int size = ch < KPL ? kcnt[ch < KPL ? ch : 0] : 0;
        if (j >= ck && j < ce) size = j == ck ? valid_text : text - valid_text;
        const int incl = wave_incl_scan(size);
        const int a = min(sk, pre + incl - size), e = min(sk, pre + incl);
        const bool has_rows = e > a;
        const bool on = has_rows && kept(j);
        const uint64_t with_rows = __ballot(has_rows), on_mask = __ballot(on);
        const uint64_t lower = with_rows & below;
        const bool prev = lower ? ((on_mask >> (63 - __builtin_clzll(lower))) & 1ull) != 0 : prev_on;
        const bool start = on && !prev;
        const uint64_t starts = __ballot(start);
        const int orows = on ? e - a : 0;
        const int oincl = wave_incl_scan(orows);
        const int off = run + oincl - orows;  // stream offset of cluster j
        if (start) srow[1 + nseg + __popcll(starts & below)] = int2{a - off, off};
        nseg += __popcll(starts);
        run += __shfl(oincl, kWave - 1, kWave);
        pre += __shfl(incl, kWave - 1, kWave);
        if (with_rows) prev_on = ((on_mask >> (63 - __builtin_clzll(with_rows))) & 1ull) != 0;
    }
    if (lane == 0) {
        srow[0] = int2{nseg, run};
        srow[1 + nseg] = int2{0, 0x7fffffff};
    }
    return run;
}

// kWork: besides (or instead of) the map, write every map row's kept-segment list and stream
// length into `work`; the last workgroup of each batch entry to finish (arrival counter) then
// orders that entry's attention items.
template <int KPL, bool kWork, bool kWide>
__global__ __launch_bounds__(kSelWaves * kWave) void select_kernel(
    const float* __restrict__ qc, const float* __restrict__ kc, const int32_t* __restrict__ qn,
    const int32_t* __restrict__ kn, int bh, int cq, int ck, int dims, float scale, float p, int minimum, int extend,
    int valid_text, int text, uint8_t* __restrict__ map, int32_t* __restrict__ ext_q, int32_t* __restrict__ ext_k,
    int32_t* __restrict__ kept_keys, int sq, int sk, SelWork work) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int groups = static_cast<int>(ceil_div(cq, kSelWaves));
    const int b = blockIdx.x / groups;
    const int c0 = (blockIdx.x % groups) * kSelWaves;
    const int c = c0 + wave;
    const bool active = c < cq;
    const int ce = extend ? ck + 2 : ck;
    const int re = extend ? cq + 2 : cq;
    const int kstride = dims + 1;
    const int qstride = (dims + 3) & ~3;                    // keeps float4 reads of a row aligned
    float* qrows = reinterpret_cast<float*>(smem);          // [kSelWaves][qstride]
    float* kblk = qrows + kSelWaves * qstride;               // [kSelBlock][dims + 1]
    uint8_t* flags = reinterpret_cast<uint8_t*>(kblk + kSelBlock * kstride) + static_cast<size_t>(wave) * ck;

    // Text partition rows and extended sizes (once per batch entry).
    if (extend && c0 == 0 && wave == 0) {
        if (map) {
            uint8_t* m = map + static_cast<int64_t>(b) * re * ce;
            for (int j = lane; j < ce; j += kWave) {
                m[static_cast<int64_t>(cq) * ce + j] = j < ck + 1;        // valid-text row: all but padding
                m[static_cast<int64_t>(cq + 1) * ce + j] = j == ck + 1;   // padding row: padding only
            }
        }
        if (ext_q)
            for (int i = lane; i < cq; i += kWave) ext_q[static_cast<int64_t>(b) * re + i] = qn[static_cast<int64_t>(b) * cq + i];
        if (ext_k)
            for (int j = lane; j < ck; j += kWave) ext_k[static_cast<int64_t>(b) * ce + j] = kn[static_cast<int64_t>(b) * ck + j];
        if (lane == 0 && ext_q && ext_k) {
            ext_q[static_cast<int64_t>(b) * re + cq] = valid_text;
            ext_q[static_cast<int64_t>(b) * re + cq + 1] = text - valid_text;
            ext_k[static_cast<int64_t>(b) * ce + ck] = valid_text;
            ext_k[static_cast<int64_t>(b) * ce + ck + 1] = text - valid_text;
        }
        if (kept_keys) {
            // The valid-text row sees every video key and the valid text; the padding row only
            // the padding.
            int all = 0;
            for (int j = lane; j < ck; j += kWave) all += max(0, kn[static_cast<int64_t>(b) * ck + j]);
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) all += __shfl_xor(all, m, kWave);
            if (lane == 0) {
                kept_keys[static_cast<int64_t>(b) * re + cq] = all + valid_text;
                kept_keys[static_cast<int64_t>(b) * re + cq + 1] = text - valid_text;
            }
        }
    }
    for (int t = threadIdx.x; t < kSelWaves * dims; t += blockDim.x) {
        const int r = c0 + t / dims;
        qrows[(t / dims) * qstride + t % dims] = r < cq ? qc[(static_cast<int64_t>(b) * cq + r) * dims + t % dims] : 0.0f;
    }
    const int32_t* kcount = kn + static_cast<int64_t>(b) * ck;
    const float* q = qrows + wave * qstride;

    // Key blocks are fetched into registers kDepth blocks ahead (all loads of a block in flight
    // at once) and stored to LDS rows of stride dims+1. Thread t handles elements t, t + 512, ...
    // of the block; (row, col) of element t advance incrementally.
    constexpr int kLoads = sel_loads<kWide>();
    constexpr int kDepth = sel_depth<KPL, kWide>();
    float staged[kDepth][kLoads];
    const int row_step = kSelThreads / dims, col_step = kSelThreads % dims;
    const int row0 = threadIdx.x / dims, col0 = threadIdx.x % dims;
    auto fetch = [&](float (&dst)[kLoads], int base) {
        const int n = min(kSelBlock, ck - base) * dims;
        const float* src = kc + (static_cast<int64_t>(b) * ck + base) * dims;
#pragma unroll
        for (int v = 0; v < kLoads; ++v) {
            const int t = v * kSelThreads + static_cast<int>(threadIdx.x);
            dst[v] = src[min(t, n - 1)];  // unconditional (clamped): all loads in flight
        }
    };
    auto store = [&](const float (&src)[kLoads], int base) {
        const int n = min(kSelBlock, ck - base) * dims;
        int row = row0, col = col0;
#pragma unroll
        for (int v = 0; v < kLoads; ++v) {
            if (v * kSelThreads + static_cast<int>(threadIdx.x) < n) kblk[row * kstride + col] = src[v];
            row += row_step;
            col += col_step;
            if (col >= dims) {
                col -= dims;
                ++row;
            }
        }
    };

    // Logits of key j = 64 e + lane in register slot e. The slots first hold log(count_j)
    // (-inf for an empty or absent key), read before any key block is prefetched.
    float logit[KPL];
    int kcnt[KPL];  // the counts again, for the segment lists
#pragma unroll
    for (int e = 0; e < KPL; ++e) {
        const int j = e * kSelBlock + lane;
        const int wl = kcount[min(j, ck - 1)];
        const int w = j < ck ? wl : 0;
        kcnt[e] = max(0, w);
        logit[e] = w > 0 ? logf(static_cast<float>(w)) : -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < kDepth; ++e)
        if (e * kSelBlock < ck) fetch(staged[e], e * kSelBlock);
    float lmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < KPL; ++e) {
        const int base = e * kSelBlock;
        if (base < ck) {
            const int rows = min(kSelBlock, ck - base);
            __syncthreads();  // the previous block is consumed (and the query rows are staged)
            store(staged[e % kDepth], base);
            __syncthreads();
            if (base + kDepth * kSelBlock < ck) fetch(staged[e % kDepth], base + kDepth * kSelBlock);
            if (active && lane < rows && logit[e] > -INFINITY) {
                const float* kr = kblk + lane * kstride;
                float dot = 0.0f;
                int d = 0;
                // Batches of kSelBatch key values are read before their fma chain so the
                // LDS reads of a batch are in flight together.
                for (; d + kSelBatch <= dims; d += kSelBatch) {
                    float kv[kSelBatch];
#pragma unroll
                    for (int i = 0; i < kSelBatch; ++i) kv[i] = kr[d + i];
#pragma unroll
                    for (int i = 0; i < kSelBatch; i += 4) {
                        const float4 q4 = *reinterpret_cast<const float4*>(q + d + i);
                        dot = fmaf(q4.x, kv[i], dot);
                        dot = fmaf(q4.y, kv[i + 1], dot);
                        dot = fmaf(q4.z, kv[i + 2], dot);
                        dot = fmaf(q4.w, kv[i + 3], dot);
                    }
                }
                for (; d < dims; ++d) dot = fmaf(q[d], kr[d], dot);
                logit[e] = dot * scale + logit[e];
            }
            lmax = fmaxf(lmax, logit[e]);
        }
    }
    if (active) {
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, m, kWave));
        if (!(lmax > -INFINITY && lmax < INFINITY)) lmax = 0.0f;
        // Masses and their sum (lane partials in index order, then a fixed xor tree).
        float part = 0.0f;
#pragma unroll
        for (int e = 0; e < KPL; ++e) {
            if (e * kSelBlock + lane < ck) {
                logit[e] = expf(logit[e] - lmax);
                part += logit[e];
            }
        }
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) part += __shfl_xor(part, m, kWave);
        const float denom = fmaxf(part, 1.17549435e-38f);
        // Sort keys (~orderable(prob), j): ascending = descending probability, then index.
        // Position i = KPL * lane + e initially holds key j = 64 e + lane.
        uint64_t key[KPL];
#pragma unroll
        for (int e = 0; e < KPL; ++e) {
            const int j = e * kSelBlock + lane;
            key[e] = j < ck ? (static_cast<uint64_t>(~orderable(logit[e] / denom)) << 32) | static_cast<uint32_t>(j)
                            : ~0ull;
        }
#pragma unroll
        for (int kk = 2; kk <= kWave * KPL; kk <<= 1) {
#pragma unroll
            for (int jj = kk >> 1; jj > 0; jj >>= 1) {
                if (jj >= KPL) {
                    const int m = jj / KPL;
                    const bool lower = (lane & m) == 0;
#pragma unroll
                    for (int e = 0; e < KPL; ++e) {
                        const bool up = ((lane * KPL + e) & kk) == 0;
                        const uint64_t other = shfl_xor_u64(key[e], m);
                        // Keys are distinct (indices differ) except the equal padding keys.
                        if ((key[e] < other) != (lower == up)) key[e] = other;
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < KPL; ++e) {
                        if ((e & jj) == 0) {
                            const bool up = ((lane * KPL + e) & kk) == 0;
                            const uint64_t x = key[e], y = key[e | jj];
                            const bool swap = (x > y) == up;
                            key[e] = swap ? y : x;
                            key[e | jj] = swap ? x : y;
                        }
                    }
                }
            }
        }
        // Length of the kept prefix: every lane walks the same sequential double sum, one
        // source lane (KPL sorted positions) per step, leaving the loop once per step.
        const int floor_keep = max(1, minimum);
        int kept = ck;
        if (!(p >= 1.0f)) {
            double run = 0.0;
            for (int l = 0; l * KPL < ck; ++l) {
                float prob[KPL];
#pragma unroll
                for (int e = 0; e < KPL; ++e)
                    prob[e] = key_prob(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key[e] >> 32), l)));
                bool fail[KPL];
#pragma unroll
                for (int e = 0; e < KPL; ++e) {
                    const int k = l * KPL + e;
                    if (k < ck) run += static_cast<double>(prob[e]);
                    const float before = static_cast<float>(run) - prob[e];
                    fail[e] = k < ck && k >= floor_keep && !(before < p);
                }
                int first = ck;
#pragma unroll
                for (int e = KPL - 1; e >= 0; --e)
                    if (fail[e]) first = l * KPL + e;
                if (first < ck) {
                    kept = first;
                    break;
                }
            }
        }
        const bool qnonempty = qn[static_cast<int64_t>(b) * cq + c] > 0;
        int kept_rows = 0;  // key rows behind this row's kept clusters
#pragma unroll
        for (int e = 0; e < KPL; ++e) {
            const int k = lane * KPL + e;
            if (k < ck) {
                const int j = static_cast<int>(key[e] & 0xffffffffu);
                const int n = kcount[j];
                const bool on = k < kept && qnonempty && n > 0;
                flags[j] = on;
                kept_rows += on ? n : 0;
            }
        }
        if (kept_keys) {
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) kept_rows += __shfl_xor(kept_rows, m, kWave);
            if (lane == 0)
                kept_keys[static_cast<int64_t>(b) * re + c] = kept_rows + (extend ? valid_text : 0);  // as the map row
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (map) {
            uint8_t* mrow = map + (static_cast<int64_t>(b) * re + c) * ce;
            for (int j = lane; j < ck; j += kWave) mrow[j] = flags[j];
            if (extend && lane < 2) mrow[ck + lane] = lane == 0;  // video rows see valid text, never padding
        }
        if constexpr (kWork) {
            // Video rows keep their selected clusters and the valid text, never the padding.
            int2* srow = work.segs + (static_cast<int64_t>(b) * re + c) * (ce + 2);
            const int rk = write_segments(srow, kcnt, ck, ce, valid_text, text, sk,
                                          [&](int j) { return j < ck ? flags[j] != 0 : j == ck; });
            if (lane == 0)
                __hip_atomic_store(work.row_keys + static_cast<int64_t>(b) * re + c, rk, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if constexpr (kWork) {
        __shared__ int tmp[kSelWaves];
        __shared__ int last;
        if (extend && c0 == 0 && wave < 2) {
            // The text rows: valid text sees every video key and the valid text, padding only
            // itself.
            const int r = cq + wave;
            int2* srow = work.segs + (static_cast<int64_t>(b) * re + r) * (ce + 2);
            const int rk = write_segments(srow, kcnt, ck, ce, valid_text, text, sk,
                                          [&](int j) { return wave == 0 ? j < ck + 1 : j == ck + 1; });
            if (lane == 0)
                __hip_atomic_store(work.row_keys + static_cast<int64_t>(b) * re + r, rk, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        // Arrival. The row lengths are the only data the last workgroup reads from the others
        // (device-coherent stores and loads); the segment lists and items reach the attention
        // through the kernel boundary. The barrier orders every wavefront's stores before the
        // counter increment, a release at agent scope, and the last workgroup acquires before
        // it reads, so the hand-over holds under the memory model, not only on the hardware's
        // in-order completion of the stores.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(work.tickets + b, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) ==
                   groups - 1;
        __syncthreads();
        if (!last) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        // Last workgroup of entry b: clamped query offsets of the extended partition and the
        // stream length of every row, then the entry's items in cost order.
        int* qoff = reinterpret_cast<int*>(smem);  // [re + 1]
        int* kept = qoff + re + 1;                 // [re]
        uint64_t* keys = reinterpret_cast<uint64_t*>(smem) + (2 * re + 2) / 2;  // [kSortCap]
        const int nt = kSelWaves * kWave;
        const int per = static_cast<int>(ceil_div(re, nt));
        const int r0 = min(re, static_cast<int>(threadIdx.x) * per), r1 = min(re, r0 + per);
        int local = 0;
        for (int r = r0; r < r1; ++r) {
            const int n = r < cq ? max(0, qn[static_cast<int64_t>(b) * cq + r])
                                 : (r == cq ? valid_text : text - valid_text);
            qoff[r] = n;
            local += n;
        }
        int total;
        int run = block_scan<kSelWaves>(local, tmp, &total);
        for (int r = r0; r < r1; ++r) {
            const int n = qoff[r];
            qoff[r] = min(sq, run);
            run += n;
        }
        if (threadIdx.x == 0) qoff[re] = min(sq, total);
        for (int r = threadIdx.x; r < re; r += nt)
            kept[r] = max(0, __hip_atomic_load(work.row_keys + static_cast<int64_t>(b) * re + r, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT));
        __syncthreads();
        order_head_items<kSelWaves>(qoff, kept, re, attention_item_rows(sq),
                                    work.items + static_cast<int64_t>(b) * work.cap * 3, work.counts + b, keys, tmp);
        if (threadIdx.x == 0) work.tickets[b] = 0;  // ready for the next call
    }
}

template <int KPL, bool kWide>
void launch_select(int blocks, size_t lds, hipStream_t stream, const float* qc, const float* kc, const int32_t* qn,
                   const int32_t* kn, int bh, int cq, int ck, int dims, float scale, float p, int minimum, int extend,
                   int valid_text, int text, uint8_t* map, int32_t* ext_q, int32_t* ext_k, int32_t* kept_keys,
                   int sq, int sk, const SelWork* work) {
    if (work)
        hipLaunchKernelGGL((select_kernel<KPL, true, kWide>), dim3(static_cast<unsigned>(blocks)), dim3(kSelWaves * kWave),
                           lds, stream, qc, kc, qn, kn, bh, cq, ck, dims, scale, p, minimum, extend, valid_text, text,
                           map, ext_q, ext_k, kept_keys, sq, sk, *work);
    else
        hipLaunchKernelGGL((select_kernel<KPL, false, kWide>), dim3(static_cast<unsigned>(blocks)), dim3(kSelWaves * kWave),
                           lds, stream, qc, kc, qn, kn, bh, cq, ck, dims, scale, p, minimum, extend, valid_text, text,
                           map, ext_q, ext_k, kept_keys, sq, sk, SelWork{});
}

// Shared host entry: validation, LDS size and the launch over the per-lane key count.
int select_launch(const float* qc, const float* kc, const int32_t* q_counts, const int32_t* k_counts, int bh, int cq,
                  int ck, int dims, float p, int minimum, int extend, int valid_text, int text, uint8_t* map,
                  int32_t* ext_q, int32_t* ext_k, int32_t* kept_keys, int sq, int sk, const SelWork* work,
                  void* stream) {
    if (!qc || !kc || !q_counts || !k_counts || bh < 1 || cq < 1 || ck < 1 || dims < 1 || dims > kSelMaxDims ||
        !(p >= 0.0f && p <= 1.0f) || minimum < 0 || (extend && (valid_text < 0 || valid_text > text)))
        return kInvalidValue;
    if (ck > kWave * 32) return kUnsupportedShape;
    const size_t qstride = (static_cast<size_t>(dims) + 3) & ~static_cast<size_t>(3);
    size_t lds = sizeof(float) * (kSelWaves * qstride + static_cast<size_t>(kSelBlock) * (dims + 1)) +
                 static_cast<size_t>(kSelWaves) * ck;
    if (work) {
        // The last workgroup of an entry reuses the LDS for its query offsets, row lengths and sort keys.
        const size_t re = static_cast<size_t>(extend ? cq + 2 : cq);
        lds = std::max(lds, sizeof(int) * (2 * re + 2) + sizeof(uint64_t) * kSortCap);
    }
    if (lds > 64 * 1024) return kUnsupportedShape;
    const int blocks = bh * static_cast<int>(ceil_div(cq, kSelWaves));
    const float scale = static_cast<float>(std::pow(static_cast<double>(dims), -0.5));
    auto* s = static_cast<hipStream_t>(stream);
    const int per_lane = static_cast<int>(ceil_div(ck, kWave));
#define PECO_SELECT_W(K, W)                                                                                     \
    launch_select<K, W>(blocks, lds, s, qc, kc, q_counts, k_counts, bh, cq, ck, dims, scale, p, minimum, extend, \
                        valid_text, text, map, ext_q, ext_k, kept_keys, sq, sk, work)
#define PECO_SELECT(K)                                                                                          \
    do {                                                                                                        \
        if (dims <= 128) PECO_SELECT_W(K, false);                                                               \
        else PECO_SELECT_W(K, true);                                                                            \
    } while (0)
    if (per_lane <= 1) PECO_SELECT(1);
    else if (per_lane <= 2) PECO_SELECT(2);
    else if (per_lane <= 4) PECO_SELECT(4);
    else if (per_lane <= 8) PECO_SELECT(8);
    else if (per_lane <= 16) PECO_SELECT(16);
    else PECO_SELECT(32);
#undef PECO_SELECT
#undef PECO_SELECT_W
    return hipGetLastError();
}

}  // namespace
}  // namespace peco

using namespace peco;

// Selection of cluster pairs, optionally extended with the text partition.
// qc [bh, cq, dims], kc [bh, ck, dims] fp32; q_counts [bh, cq], k_counts [bh, ck] int32.
// map: bool [bh, cq(+2), ck(+2)]; ext_q/ext_k (extend only): int32 [bh, cq+2] / [bh, ck+2].
// kept_keys (nullable): int32 [bh, cq(+2)], the number of key rows each map row keeps.
// minimum = ceil(min_kc_ratio * ck) computed by the caller. ck <= 2048, dims <= 256; the LDS use
// (8 query rows, a 64-row key block and 8 rows of ck flag bytes) must fit in 64 KiB.
PECO_API int peco_select_cluster_connections(const float* qc, const float* kc, const int32_t* q_counts,
                                             const int32_t* k_counts, int bh, int cq, int ck, int dims, float p,
                                             int minimum, int extend, int valid_text, int text, uint8_t* map,
                                             int32_t* ext_q, int32_t* ext_k, int32_t* kept_keys, void* stream) {
    if (!map || (extend && (!ext_q || !ext_k))) return kInvalidValue;
    return select_launch(qc, kc, q_counts, k_counts, bh, cq, ck, dims, p, minimum, extend, valid_text, text, map,
                         ext_q, ext_k, kept_keys, 0, 0, nullptr, stream);
}

// int32 elements of the work buffer of peco_select_work for bh entries, sq query rows and a
// (cq(+2)) x (ck(+2)) map.
PECO_API size_t peco_select_work_size(int bh, int sq, int cq, int ck, int extend) {
    if (bh < 1 || sq < 0 || cq < 1 || ck < 1) return 0;
    return sel_work_ints(bh, sq, extend ? cq + 2 : cq, extend ? ck + 2 : ck);
}

// Selection plus the attention's work list in one launch. Same selection as
// peco_select_cluster_connections (map, ext_q and ext_k optional here), and in `work`
// (peco_select_work_size int32, 8-byte aligned; the first bh of them zero before the first
// call, and every call leaves them zero) the kept-segment list and stream length of every map row and the items
// of every entry in cost order, which peco_sparse_attention_work consumes. sq and sk are the
// query and key lengths of the attention (video + text); key cluster rows are clamped to sk
// and query cluster rows to sq as the attention's own builder does.
PECO_API int peco_select_work(const float* qc, const float* kc, const int32_t* q_counts, const int32_t* k_counts,
                              int bh, int cq, int ck, int dims, float p, int minimum, int extend, int valid_text,
                              int text, int sq, int sk, uint8_t* map, int32_t* ext_q, int32_t* ext_k, int32_t* work,
                              size_t work_ints, void* stream) {
    if (!work || sq < 0 || sk < 0 || bh < 1 || cq < 1 || ck < 1) return kInvalidValue;
    const int re = extend ? cq + 2 : cq, ce = extend ? ck + 2 : ck;
    if (work_ints < sel_work_ints(bh, sq, re, ce)) return kWorkspaceTooSmall;
    const SelWork w = sel_work_layout(work, bh, sq, re, ce);
    return select_launch(qc, kc, q_counts, k_counts, bh, cq, ck, dims, p, minimum, extend, valid_text, text, map,
                         ext_q, ext_k, nullptr, sq, sk, &w, stream);
}
