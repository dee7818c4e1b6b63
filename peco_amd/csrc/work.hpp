// Attention work list: per head, the items (query-row chunks of one query cluster) ordered
// by cost, and, for the selection-built list, each map row's kept-segment list.
//
// Two producers write it:
//   - build_work_kernel (attention.hip) from a bool map and the cluster sizes, the reference
//     ABI's input (peco/kernels/sparse_attention.cu:17-46 builds its work map the same way,
//     one query tile at a time);
//   - the selection launch (select.hip, peco_select_work), which writes the kept-segment list
//     of every map row while it selects, and whose last workgroup of each head orders that
//     head's items, so no map is read and no builder launch is needed.
// Both order items with order_head_items below, so the attention sees the same list.
#pragma once

#include "common.hpp"

namespace peco {

constexpr int kQTile = 128;    // query rows per item of a 4-wavefront attention workgroup
constexpr int kSortCap = 2048; // items per head ordered by cost (more: cluster order)
constexpr int kItemBits = 12;  // sort payload: query cluster (high bits), item within it (low)

// Long sequences (at least kLongItemsFrom query rows) cut their query clusters into items of
// 2 * kQTile rows, run by 8-wavefront attention workgroups (one per CU): each K/V tile then
// serves twice the query rows, halving the tile loads per row (their clusters mostly exceed 128
// rows). Measured: the 720p attention (119056 rows) 1.7% faster, the 544p one (32896 rows) 1.3%
// slower, where one workgroup per CU hides less of the loads' latency than two. The
// work-list builders and the attention launch use this one rule, which depends on the query
// length alone, so a work list always meets the workgroups it was cut for.
constexpr int kLongItemsFrom = 65536;
__host__ __device__ inline int attention_item_rows(int sq) {
    return sq >= kLongItemsFrom ? 2 * kQTile : kQTile;
}

// Item slots per head: enough for items of kQTile rows (longer items need fewer).
__host__ __device__ inline int item_capacity(int sq, int cq) {
    return static_cast<int>(ceil_div(sq, kQTile)) + min(cq, sq);
}

// Selection-built work list, in one int32 buffer:
//   tickets int32 [bh]: arrival counters of the selection's workgroups; zero before the first
//         call on a buffer, and every call leaves them zero;
//   counts int32 [bh]: items per head;
//   row_keys int32 [bh, re]: the stream length L of every map row;
//   items int32 [bh, cap, 3]: q_start, query cluster, rows (<= kQTile), by descending cost;
//   queues int32 [kQueueInts]: the attention's item queue counters (one per XCD) and its exit
//         counter; zero before the first call, and every attention call leaves them zero;
//   segs  int2 [bh, re, ce + 2] (8-byte aligned): per map row {segment count n, L}, then n
//         segments {first physical row - stream offset, stream offset} of its kept key rows
//         (adjacent kept clusters merged), then the sentinel {0, INT_MAX}.
struct SelWork {
    int32_t* tickets;
    int32_t* counts;
    int32_t* row_keys;
    int32_t* items;
    int32_t* queues;
    int2* segs;
    int cap;
};

constexpr int kItemQueues = 8;   // attention item queues, one per XCD
constexpr int kQueueInts = 16;   // the queues' counters and the exit counter, padded

__host__ __device__ inline size_t sel_work_head_ints(int bh, int sq, int re) {
    const size_t b = static_cast<size_t>(bh);
    const size_t n = 2 * b + b * re + b * item_capacity(sq, re) * 3 + kQueueInts;
    return (n + 1) & ~static_cast<size_t>(1);
}

__host__ __device__ inline size_t sel_work_ints(int bh, int sq, int re, int ce) {
    return sel_work_head_ints(bh, sq, re) + static_cast<size_t>(bh) * re * (static_cast<size_t>(ce) + 2) * 2;
}

__host__ __device__ inline SelWork sel_work_layout(int32_t* base, int bh, int sq, int re, int ce) {
    (void)ce;
    SelWork w;
    w.cap = item_capacity(sq, re);
    w.tickets = base;
    w.counts = base + bh;
    w.row_keys = w.counts + bh;
    w.items = w.row_keys + static_cast<size_t>(bh) * re;
    w.queues = w.items + static_cast<size_t>(bh) * w.cap * 3;
    w.segs = reinterpret_cast<int2*>(base + sel_work_head_ints(bh, sq, re));
    return w;
}

__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int y = __shfl_up(v, d, kWave);
        if (lane >= d) v += y;
    }
    return v;
}

// Exclusive scan over a workgroup of NW wavefronts (sum of all values in *total). tmp holds
// NW ints of LDS. Every thread of the workgroup must call it.
template <int NW>
__device__ __forceinline__ int block_scan(int v, int* tmp, int* total) {
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int inc = wave_incl_scan(v);
    __syncthreads();
    if (lane == kWave - 1) tmp[wave] = inc;
    __syncthreads();
    int base = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        base += w < wave ? tmp[w] : 0;
        sum += tmp[w];
    }
    *total = sum;
    return base + inc - v;
}

// Items of one head from its clamped query offsets qoff[cq + 1] and the key rows each query
// cluster keeps (kept[cq]), both in LDS: every cluster is cut into items of at most `tile`
// rows (attention_item_rows), ordered by descending cost rows * kept (ties keep cluster order,
// and the chunks of a cluster stay in row order) when at most kSortCap items fit the sort,
// else in cluster order. keys: LDS for the sort, 8 bytes x (the power of two >= kSortCap).
// Every thread of the NW-wave workgroup calls it.
template <int NW>
__device__ void order_head_items(const int* qoff, const int* kept, int cq, int tile, int32_t* items,
                                 int32_t* count_out, uint64_t* keys, int* tmp) {
    constexpr int NT = NW * kWave;
    const int per = static_cast<int>(ceil_div(cq, NT));
    const int c0 = min(cq, static_cast<int>(threadIdx.x) * per), c1 = min(cq, c0 + per);
    int local = 0;
    bool fits = true;  // every item is addressable by the sort payload
    for (int c = c0; c < c1; ++c) {
        const int n = static_cast<int>(ceil_div(qoff[c + 1] - qoff[c], tile));
        local += n;
        fits = fits && n <= (1 << kItemBits);
    }
    int count;
    int slot = block_scan<NW>(local, tmp, &count);
    const bool sortable = count <= kSortCap && __syncthreads_and(fits) && cq < (1 << (32 - kItemBits));
    if (threadIdx.x == 0) *count_out = count;
    if (!sortable) {
        for (int c = c0; c < c1; ++c) {
            const int rows = qoff[c + 1] - qoff[c];
            for (int r = 0; r < rows; r += tile, ++slot) {
                items[3 * slot + 0] = qoff[c] + r;
                items[3 * slot + 1] = c;
                items[3 * slot + 2] = min(tile, rows - r);
            }
        }
        return;
    }
    for (int c = c0; c < c1; ++c) {
        const int rows = qoff[c + 1] - qoff[c];
        for (int r = 0, ri = 0; r < rows; r += tile, ++slot, ++ri) {
            const int n = min(tile, rows - r);
            const uint32_t cost = static_cast<uint32_t>(min<int64_t>(static_cast<int64_t>(n) * kept[c], 0x7fffffff));
            // (descending cost, cluster, item) for an ascending sort.
            keys[slot] = (static_cast<uint64_t>(~cost) << 32) | (static_cast<uint32_t>(c) << kItemBits) |
                         static_cast<uint32_t>(ri);
        }
    }
    __syncthreads();
    auto emit = [&](int pos, uint64_t key) {
        const uint32_t payload = static_cast<uint32_t>(key);
        const int c = static_cast<int>(payload >> kItemBits);
        const int r = static_cast<int>(payload & ((1u << kItemBits) - 1u)) * tile;
        items[3 * pos + 0] = qoff[c] + r;
        items[3 * pos + 1] = c;
        items[3 * pos + 2] = min(tile, qoff[c + 1] - qoff[c] - r);
    };
    if (count <= NT) {
        // Rank sort: the keys are distinct, so each one's rank (the number of smaller keys) is
        // its position. All threads read the same key at a time (LDS broadcast).
        const uint64_t mine = static_cast<int>(threadIdx.x) < count ? keys[threadIdx.x] : ~0ull;
        int rank = 0;
        for (int j = 0; j < count; ++j) rank += keys[j] < mine ? 1 : 0;
        if (static_cast<int>(threadIdx.x) < count) emit(rank, mine);
        return;
    }
    int n2 = 1;
    while (n2 < count) n2 <<= 1;
    for (int i = count + threadIdx.x; i < n2; i += NT) keys[i] = ~0ull;
    __syncthreads();
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n2; i += NT) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = keys[i], b = keys[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        keys[i] = b;
                        keys[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < count; i += NT) emit(i, keys[i]);
}

}  // namespace peco
