// Stage 4: cluster-sparse flash attention on MFMA (gfx950), with its device work list.
//
// Semantics (peco/attention_cuda.py:75-83, peco/kernels/sparse_attention.cu:17-46,94,135-158,187):
//   out_i = sum_{j : map[cq(i), ck(j)]} softmax_j(q_i.k_j / sqrt(D)) v_j, and 0 when row i
//   keeps no key. Query and key rows are grouped by cluster in the order of q_sizes/k_sizes.
//
// Work list (one 256-thread workgroup per (batch*head)):
//   cluster offsets are min(S, prefix of max(0, size)) (the reference's clamped running sum),
//   each query cluster is cut into items of <= 128 rows (256 from 65536 query rows on), and the
//   items of one head are ordered by descending cost rows * kept_keys. The attention grid is
//   slot-major over bands
//   of heads (block = band_index * band * cap + slot * band + head in band): the costliest
//   item of every head of a band starts first. The band is all heads when their K/V take at
//   most 96 MB (then, with BH a multiple of 8, all items of one head land on one XCD, whose L2
//   holds that head's K/V), else up to four heads whose K/V fit in the MALL, so long
//   sequences re-read each head's K/V from the MALL instead of HBM.
//
// Attention workgroup = one item: 4 waves x 32 query rows (8 waves x 32 rows for the 256-row
// items of long sequences, see attention_item_rows in work.hpp). The kept key clusters of the
// item's query cluster form one virtual key stream (their rows are contiguous per cluster
// after the sort); it is processed in 64-key tiles gathered into LDS, so ragged clusters
// cost no masked MFMA work except the stream's last partial tile.
//   S^T = K Q^T  (v_mfma_f32_32x32x16, A = K tile from LDS, B = Q^T held in VGPRs):
//         lane l holds query l%32 and keys 8*(i/4) + 4*(l/32) + i%4,
//   online softmax in fp32 with exp2 (v_exp_f32), per-query state per lane,
//   O^T += V^T P^T (A = V^T from a transposed LDS tile, B = P^T straight from the S^T
//         accumulators rounded to bf16/fp16, no shuffle needed).
// P is rounded to the input dtype before the PV product (the reference keeps P in fp32).
// An optional out_index writes each output row straight to its original sequence position
// (fusing restore_sequence_order, peco/clustering.py:128-136).
#include "base_offset.hpp"
#include "common.hpp"
#include "work.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace peco {
namespace {

constexpr int kKTile = 64;    // keys per LDS tile

struct WorkLayout {
    int32_t* counts;   // [bh]
    int32_t* kprefix;  // [bh, ck + 1]
    int32_t* items;    // [bh, cap, 3]: q_start, q_cluster, q_rows
    int cap;
};

__host__ __device__ inline WorkLayout work_layout(int32_t* ws, int bh, int sq, int cq, int ck) {
    WorkLayout w;
    w.cap = item_capacity(sq, cq);
    w.counts = ws;
    w.kprefix = ws + bh;
    w.items = w.kprefix + static_cast<int64_t>(bh) * (ck + 1);
    return w;
}

// Map rows read per wavefront per pass, and bytes of a row per lane per pass (320 keys): one
// pass covers a head of up to 96 query clusters and 320 key clusters.
constexpr int kMapRows = 24;
constexpr int kMapU = 5;

// kGivenKept: kept_in [bh, cq] holds each query cluster's kept key rows (from the selection
// launch), so the map is not read; the counts only order the items.
template <bool kGivenKept>
__global__ __launch_bounds__(256) void build_work_kernel(const uint8_t* __restrict__ selected,
                                                         const int* __restrict__ q_sizes,
                                                         const int* __restrict__ k_sizes,
                                                         const int32_t* __restrict__ kept_in, int32_t* ws, int bhn,
                                                         int sq, int sk, int cq, int ck, int tile) {
    extern __shared__ int lds[];
    __shared__ int tmp[4];
    const int bh = blockIdx.x;
    const int wave = threadIdx.x / kWave, lane = lane_id();
    WorkLayout W = work_layout(ws, bhn, sq, cq, ck);
    int* ksz = lds;              // [ck] clamped key cluster sizes
    int* qoff = ksz + ck;        // [cq + 1] clamped query offsets
    int* kept = qoff + cq + 1;   // [cq] kept keys per query cluster
    uint64_t* keys = reinterpret_cast<uint64_t*>(lds + ((ck + 2 * cq + 1 + 1) & ~1));  // [pow2 >= cap] sort keys
    int32_t* kpre = W.kprefix + static_cast<int64_t>(bh) * (ck + 1);
    const uint8_t* map = selected + static_cast<int64_t>(bh) * cq * ck;
    // The map rows of wavefront w are w, w+4, ...; a pass covers kMapRows of them and kMapU*64
    // keys, every byte load of the pass in flight at once. The first pass is issued before the
    // size scans so its latency overlaps them.
    const int my_rows = cq > wave ? static_cast<int>(ceil_div(cq - wave, 4)) : 0;
    const int chunks = static_cast<int>(ceil_div(ck, kMapU * kWave));
    const int passes = kGivenKept ? 0 : static_cast<int>(ceil_div(my_rows, kMapRows)) * chunks;
    // Raw bytes, kept unmasked so that the loads stay in flight until the pass uses them: a
    // clamped duplicate row (past my_rows) is never written back, a clamped column (past ck)
    // meets a zero size.
    int m[kMapRows][kMapU];
    auto issue = [&](int pass) {
        const int r0 = (pass / chunks) * kMapRows;
        const int k0 = (pass % chunks) * kMapU * kWave;
#pragma unroll
        for (int r = 0; r < kMapRows; ++r) {
            const int c = min(wave + 4 * max(0, min(r0 + r, my_rows - 1)), cq - 1);
            const uint8_t* row = map + static_cast<int64_t>(c) * ck;
#pragma unroll
            for (int u = 0; u < kMapU; ++u) m[r][u] = row[min(k0 + u * kWave + lane, ck - 1)];
        }
    };
    // Cluster sizes: up to kSizes per thread are loaded together (clamped, masked after). They
    // are issued before the first map pass: loads complete in order, so the size scans below
    // then wait only for these.
    constexpr int kSizes = 4;
    const int kper = static_cast<int>(ceil_div(ck, 256));
    const int qper = static_cast<int>(ceil_div(cq, 256));
    int kv[kSizes], qv[kSizes];
    if (kper <= kSizes && qper <= kSizes) {
#pragma unroll
        for (int i = 0; i < kSizes; ++i) {
            kv[i] = k_sizes[static_cast<int64_t>(bh) * ck + min(static_cast<int>(threadIdx.x) * kper + i, ck - 1)];
            qv[i] = q_sizes[static_cast<int64_t>(bh) * cq + min(static_cast<int>(threadIdx.x) * qper + i, cq - 1)];
        }
    }
    if constexpr (!kGivenKept) issue(0);  // unconditional (rows clamped): later waits count these loads exactly
    for (int c = threadIdx.x; c < cq; c += blockDim.x)
        kept[c] = kGivenKept ? max(0, kept_in[static_cast<int64_t>(bh) * cq + c]) : 0;
    // Key cluster offsets: min(sk, prefix of max(0, size)).
    {
        const int per = kper;
        const int c0 = threadIdx.x * per, c1 = min(ck, c0 + per);
        int local = 0;
        if (kper <= kSizes && qper <= kSizes) {
#pragma unroll
            for (int i = 0; i < kSizes; ++i) {
                if (c0 + i < c1) {
                    ksz[c0 + i] = max(0, kv[i]);
                    local += max(0, kv[i]);
                }
            }
        } else {
            for (int c = c0; c < c1; ++c) {
                const int v = max(0, k_sizes[static_cast<int64_t>(bh) * ck + c]);
                ksz[c] = v;
                local += v;
            }
        }
        int total;
        int run = block_scan<4>(local, tmp, &total);
        for (int c = c0; c < c1; ++c) {
            const int a = min(sk, run);
            run += ksz[c];
            const int e = min(sk, run);
            kpre[c] = a;
            ksz[c] = e - a;
        }
        if (threadIdx.x == 0) kpre[ck] = min(sk, total);
    }
    // Query cluster offsets (qoff[c] holds the clamped size until the scan replaces it).
    {
        const int per = qper;
        const int c0 = threadIdx.x * per, c1 = min(cq, c0 + per);
        int local = 0;
        if (kper <= kSizes && qper <= kSizes) {
#pragma unroll
            for (int i = 0; i < kSizes; ++i) {
                if (c0 + i < c1) {
                    qoff[c0 + i] = max(0, qv[i]);
                    local += max(0, qv[i]);
                }
            }
        } else {
            for (int c = c0; c < c1; ++c) {
                const int v = max(0, q_sizes[static_cast<int64_t>(bh) * cq + c]);
                qoff[c] = v;
                local += v;
            }
        }
        int total;
        int run = block_scan<4>(local, tmp, &total);
        for (int c = c0; c < c1; ++c) {
            const int v = qoff[c];
            qoff[c] = min(sq, run);
            run += v;
        }
        if (threadIdx.x == 0) qoff[cq] = min(sq, total);
    }
    __syncthreads();
    // Kept keys per query cluster: each pass adds its rows' chunk sums (a row is only ever
    // touched by its own wavefront, so the read-modify-write needs no atomics).
    for (int pass = 0; pass < passes; ++pass) {
        const int r0 = (pass / chunks) * kMapRows;
        const int k0 = (pass % chunks) * kMapU * kWave;
        int w[kMapU];  // sizes of this lane's key clusters in the chunk (0 past ck)
#pragma unroll
        for (int u = 0; u < kMapU; ++u) {
            const int kc = k0 + u * kWave + lane;
            const int v = ksz[min(kc, ck - 1)];
            w[u] = kc < ck ? v : 0;
        }
        int sum[kMapRows];
#pragma unroll
        for (int r = 0; r < kMapRows; ++r) {
            sum[r] = 0;
#pragma unroll
            for (int u = 0; u < kMapU; ++u) sum[r] += (m[r][u] & 0xff) ? w[u] : 0;
        }
        if (pass + 1 < passes) issue(pass + 1);
#pragma unroll
        for (int r = 0; r < kMapRows; ++r) {
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) sum[r] += __shfl_xor(sum[r], o, kWave);
            if (lane == 0 && r0 + r < my_rows) kept[wave + 4 * (r0 + r)] += sum[r];
        }
    }
    __syncthreads();
    order_head_items<4>(qoff, kept, cq, tile, W.items + static_cast<int64_t>(bh) * W.cap * 3, W.counts + bh, keys,
                        tmp);
}

template <int DT> struct Mfma;
template <> struct Mfma<kBF16> {
    static __device__ __forceinline__ f32x16 run(u16x8 a, u16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    }
    // Two fp32 -> packed pair with round-to-nearest-even (v_cvt_pk_bf16_f32).
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));
    }
    // acc + lo(p) + hi(p) of a packed pair (v_dot2_f32_bf16 against (1, 1)).
    static __device__ __forceinline__ float sum2(uint32_t p, float acc) {
        typedef __bf16 b2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, p), __builtin_bit_cast(b2, 0x3f803f80u), acc,
                                               false);
    }
};
template <> struct Mfma<kF16> {
    static __device__ __forceinline__ f32x16 run(u16x8 a, u16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
    }
    static __device__ __forceinline__ float sum2(uint32_t p, float acc) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, p), __builtin_bit_cast(h2, 0x3c003c00u), acc, false);
    }
};

// K and V tiles live in LDS row-major ([64 keys][D], no padding) and are filled straight
// from global memory with 16-byte global_load_lds, which writes each wave's 64 lanes to one
// contiguous 1 KB span. Bank conflicts are avoided by XOR-swizzling the 16-byte chunks of a
// row: a lane whose LDS slot is (row, physical chunk p) fetches logical chunk p ^ swz(row).
//   K: swz = row % CH, so the 16 rows read by one S^T A-fragment quarter-wave hit 16 chunks.
//   V: swz spreads the 4 rows x 32 bytes of one transpose read over distinct banks.
template <int D> struct Tiles {
    static constexpr int CH = D / 8;                  // 16-byte chunks per row
    static constexpr int kElems = kKTile * D;
    static constexpr int kWaveRows = kWave / CH;      // rows per wave-wide direct load
    static constexpr int kLoads = kKTile / (4 * kWaveRows);  // direct loads per wave per tile
    static __device__ __forceinline__ int swz_k(int row) { return row % CH; }
    static __device__ __forceinline__ int swz_v(int row) { return CH == 16 ? 4 * (row % 4) : 4 * ((row >> 1) & 1); }
};



// Issue the direct-to-LDS loads of one K and one V tile (no wait), or the share of a wave
// that is one of NL loaders (rank `first`): the tile's 4*kLoads spans of 64 lanes x 16 bytes
// per tensor go round-robin to the loaders. Rows past the stream end read row 0 of the head:
// their K scores are masked to -inf and their P is 0.
template <int D, int NL>
__device__ __forceinline__ void load_tile_lds(uint16_t* ks, uint16_t* vs, const uint16_t* kh, const uint16_t* vh,
                                              const int* prow, int first, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
    using T = Tiles<D>;
    constexpr int kSpans = 4 * T::kLoads / NL;  // spans per tensor for this loader
    constexpr int kGroup = kSpans < 4 ? kSpans : 4;  // spans whose rows are read at once
    // LDS byte address of this loader's first span in the K tile (wave-uniform) and the distance
    // from a K span to the matching V span.
    const uint32_t lds_base = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ks + first * kWave * 8)));
    const uint32_t vs_delta = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>(vs) - reinterpret_cast<uintptr_t>(ks)));
#pragma unroll 1
    for (int i0 = 0; i0 < kSpans; i0 += kGroup) {
        int rows[kGroup];
#pragma unroll
        for (int j = 0; j < kGroup; ++j) rows[j] = prow[((i0 + j) * NL + first) * T::kWaveRows + lane / T::CH];
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            const int i = i0 + j;
            const int r = (i * NL + first) * T::kWaveRows + lane / T::CH;  // tile row written by this lane
            const int p = lane % T::CH;                                        // physical chunk
            // Byte offsets within the head (rows < 2^31 / (2 D) there, so 32 bits suffice).
            const uint32_t g = static_cast<uint32_t>(rows[j]) * (D * 2);
            const uint32_t kdst = lds_base + static_cast<uint32_t>(((i * NL) * kWave * 8) * 2);
            const uint32_t vdst = kdst + vs_delta;
            dma16_off(kh, g + (p ^ T::swz_k(r)) * 16, kdst);
            dma16_off(vh, g + (p ^ T::swz_v(r)) * 16, vdst);
        }
    }
#endif
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Input modes:
//   kPacked: Q, K and V in cluster order (out_index, when given, only scatters the output);
//   kIndexed: the inputs are in their original token order. Query row j < oi_rows of a head
//     is read from row out_index[j] (the same permutation that scatters the output) and
//     key/value stream row p < oi_rows from row k_index[p]; rows past oi_rows (text) keep
//     their position;
//   kQuantQ: K and V in cluster order, Q in original order read through out_index as in
//     kIndexed and Base-Offset fake-quantized as it is loaded: every row of an item belongs
//     to its query cluster qc, so rows of a video cluster (qc < qcent_rows) take centroid
//     qcent[bh, qc] and levels = 2^bits - 1 (peco/processor.py:141, fused into the load);
//   kIndexedQuantQ: Q as in kQuantQ, K and V in original order read through k_index as in
//     kIndexed (the Base-Offset layer: K fake-quantized in original order by the fit, V the
//     caller's own tensor).
// The key stream of an item comes either from a kept-segment list (segs, as the selection
// launch writes it: {count n, stream length L}, n segments, sentinel per map row) or, when segs
// is null, from the item's map row and the clamped key-cluster prefix kprefix [bh, ck + 1].
enum InputMode : int { kPacked = 0, kIndexed = 1, kQuantQ = 2, kIndexedQuantQ = 3 };

// One work item (linear index g over bands x slots x heads, see below) of the attention, run
// by a workgroup of kWaves wavefronts (4, or 8 for the items of 2 * kQTile rows).
template <int DT, int D, int kMode, int kWaves>
__device__ __forceinline__ void attention_item(
    int g, const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint8_t* __restrict__ selected, const int32_t* __restrict__ kprefix, const int2* __restrict__ segs,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ items, int cap, uint16_t* __restrict__ out,
    const int32_t* __restrict__ out_index, int oi_rows, const int32_t* __restrict__ k_index,
    const float* __restrict__ qcent, int qcent_rows, float levels, int bhn, int band, int sq, int sk, int cq,
    int ck, float scale_log2) {
    constexpr bool kIndexedKV = kMode == kIndexed || kMode == kIndexedQuantQ;
    constexpr bool kQuantLoad = kMode == kQuantQ || kMode == kIndexedQuantQ;
    using T = Tiles<D>;
    constexpr int S = D / 16;       // k-steps of S^T over channels
    constexpr int NB = D / 32;      // 32-channel blocks of O^T
    // Scores may run up to 2^8 above the running maximum before O is rescaled.
    constexpr float kLazyLog2 = 8.0f;
    // K tiles (buffers 0, 1) and V tiles (2, 3) in one array: after the last tile the paired
    // waves exchange their softmax states through it, which takes more than the K half.
    constexpr int NT = kWaves * kWave;           // threads of the workgroup
    constexpr int H = kWaves / 2;                // row blocks of a paired (split) item
    constexpr int kRowsPerWave = kKTile / kWaves;  // tile rows whose physical row a wave looks up
    __shared__ __align__(16) uint16_t kvs[4][T::kElems];
    uint16_t(*const ks)[T::kElems] = kvs;
    uint16_t(*const vs)[T::kElems] = kvs + 2;
    static_assert(2 * kWave * (NB * 16 + 2) * sizeof(float) <= sizeof(kvs), "pair exchange exceeds the tile LDS");
    __shared__ int prow[2][kKTile];
    __shared__ int pidx[2][kKTile];    // k_index values of tile t+3 rows (indexed inputs)
    __shared__ int tmp[kWaves];
    extern __shared__ int dyn[];
    // Key stream of this query cluster: the kept, non-empty key clusters in order. Segment i
    // is {first physical row - stream offset, stream offset} of the i-th of them, followed by
    // a sentinel whose offset no stream row reaches.
    int2* kseg = reinterpret_cast<int2*>(dyn);  // [ck + 1]

    // Heads run in bands of `band` (a divisor of bhn), slot-major within a band.
    const int per_band = band * cap;
    const int in_band = g % per_band;
    const int bh = (g / per_band) * band + in_band % band;
    const int slot = in_band / band;
    if (slot >= counts[bh]) return;
    const int32_t* item = items + (static_cast<int64_t>(bh) * cap + slot) * 3;
    // Values every lane loads alike are moved to scalar registers (readfirstlane), so the
    // branches on them are wave-uniform.
    const int q_start = __builtin_amdgcn_readfirstlane(item[0]);
    const int qc = __builtin_amdgcn_readfirstlane(item[1]);
    const int q_rows = __builtin_amdgcn_readfirstlane(item[2]);
    const int tid = threadIdx.x, lane = tid % kWave, h = lane / 32;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int64_t head = static_cast<int64_t>(bh);
    const uint32_t sq_last = static_cast<uint32_t>(sq - 1), sk_last = static_cast<uint32_t>(sk - 1);

    // Items of at most 32 * H rows pair the waves: wave w takes 32-row block w % H and, of
    // every tile, only the 32-key half w / H, so a short item's tiles cost about half the
    // time; each pair merges its two partial softmax states after the last tile. Longer items
    // give each wave its own row block and both halves of every tile.
    const bool split = q_rows <= 32 * H;
    const int rb = split ? (wave % H) : wave;  // this wave's 32-row block
    const int hb = split ? (wave / H) : 0;     // first 32-key half this wave processes
    // Waves without query rows issue every tile load, so that waiting for the load path to
    // accept them never delays a wave with MFMA work; with no such wave all of them share.
    const int row_blocks = static_cast<int>(ceil_div(q_rows, 32));
    const int idle = split ? kWaves - 2 * row_blocks : kWaves - row_blocks;
    const int loaders = idle >= 4 ? 4 : (idle >= 2 ? 2 : (idle == 1 ? 1 : kWaves));
    int loader_rank;
    if (loaders == kWaves) {
        loader_rank = wave;
    } else if (split) {
        // Idle waves hold row blocks row_blocks .. H-1 of either key half.
        const int r = rb >= row_blocks ? (wave / H) * (H - row_blocks) + (rb - row_blocks) : -1;
        loader_rank = r < loaders ? r : -1;
    } else {
        loader_rank = wave >= kWaves - loaders ? wave - (kWaves - loaders) : -1;
    }
    // Q^T operand: lane holds query row (32*rb + l%32), channels 16s + 8h .. +7. Its loads
    // (and the permutation entry they depend on) go out before the key stream's, so their
    // latency overlaps the stream setup below.
    const int qrow = rb * 32 + (lane % 32);
    const bool qvalid = qrow < q_rows;
    const bool wave_active = rb * 32 < q_rows;
    int64_t qsrc = q_start + qrow;
    if constexpr (kMode != kPacked) {
        if (qvalid && qsrc < oi_rows) qsrc = min(static_cast<uint32_t>(out_index[head * oi_rows + qsrc]), sq_last);
    }
    // The segment list's header and first 256 entries (the row holds ck + 2 entries, so the
    // clamped load stays inside it) are requested before the query rows, which wait for the
    // permutation entry.
    const int2* srow = segs ? segs + (static_cast<int64_t>(bh) * cq + qc) * (ck + 2) : nullptr;
    int2 hdr{0, 0}, first{0, 0};
    if (segs) {
        hdr = srow[0];
        first = srow[1 + min(tid, ck)];
    }
    u16x8 qf[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        qf[s] = qvalid ? *reinterpret_cast<const u16x8*>(q + (head * sq + qsrc) * D + 16 * s + 8 * h)
                       : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    // kQuantQ: the centroid channels of this lane's half row (every row of the item has the
    // item's query cluster), requested with the rows.
    f32x8 qc_row[kQuantLoad ? S : 1];
    if constexpr (kQuantLoad) {
        const float* crow = qcent + (head * qcent_rows + min(qc, qcent_rows - 1)) * D + 8 * h;
#pragma unroll
        for (int s = 0; s < S; ++s) qc_row[s] = *reinterpret_cast<const f32x8*>(crow + 16 * s);
    }
    int L, nk;
    if (segs) {
        nk = min(max(hdr.x, 0), ck);
        L = max(hdr.y, 0);
        if (tid <= nk) kseg[tid] = first;
        for (int i = tid + NT; i <= nk; i += NT) kseg[i] = srow[1 + i];
    } else {
        const uint8_t* sel = selected + (static_cast<int64_t>(bh) * cq + qc) * ck;
        const int32_t* gk = kprefix + static_cast<int64_t>(bh) * (ck + 1);
        const int per = static_cast<int>(ceil_div(ck, NT));
        const int c0 = tid * per, c1 = min(ck, c0 + per);
        int local = 0, lcount = 0;
        for (int c = c0; c < c1; ++c) {
            const int a = gk[c], e = gk[c + 1];
            if (sel[c] && e > a) {
                local += e - a;
                ++lcount;
            }
        }
        int run = block_scan<kWaves>(local, tmp, &L);
        int idx = block_scan<kWaves>(lcount, tmp, &nk);
        for (int c = c0; c < c1; ++c) {
            const int a = gk[c], e = gk[c + 1];
            if (sel[c] && e > a) {
                kseg[idx] = int2{a - run, run};
                ++idx;
                run += e - a;
            }
        }
        if (tid == 0) kseg[nk] = int2{0, 0x7fffffff};
    }
    __syncthreads();
    L = __builtin_amdgcn_readfirstlane(L);
    nk = __builtin_amdgcn_readfirstlane(nk);
    const int ntiles = static_cast<int>(ceil_div(L, kKTile));
    // Physical row of stream row r (r < L). Every lane asks for increasing rows (its row of
    // every tile), so a forward-only cursor over the segments suffices.
    // The current segment's row delta and end stay in registers; the segment table is read
    // only when a row crosses into a later segment.
    int cur = 0, seg_x = kseg[0].x, seg_end = nk > 0 ? kseg[1].y : 0x7fffffff;
    auto row_of = [&](int r) {
        while (seg_end <= r) {
            ++cur;
            seg_x = kseg[cur].x;
            seg_end = kseg[cur + 1].y;
        }
        return r + seg_x;
    };
    // Tile rows move through a pipeline. Lane l of wave w follows tile row 16*w + l%16 (lanes
    // 0..15 own it, the others shadow it). During tile t it issues the direct-to-LDS loads of
    // tile t+1 (rows in prow, written a tile earlier) right after its S^T MFMAs; at the end,
    // off the MFMAs' path, it looks up its tile t+2 row and publishes it in prow. Indexed
    // inputs look two tiles further: the k_index value of the tile t+3 row is loaded straight
    // into pidx at the end of tile t and used at the end of tile t+1. Every load of the loop
    // goes straight to LDS (no register is written behind the compiler's back), so the loop
    // waits for them explicitly.
    const int32_t* kidx = kIndexedKV ? k_index + head * oi_rows : nullptr;
    const int prow_entry = kRowsPerWave * wave + lane % kRowsPerWave;
    const bool prow_owner = lane < kRowsPerWave;
    // Stream position (cluster-order row) of stream row r; rows past the stream read row 0.
    auto stream_pos = [&](int r) { return r < L ? static_cast<int>(min(static_cast<uint32_t>(row_of(r)), sk_last)) : 0; };
    // Physical row of stream position p, given k_index[p] (clamped to the head's rows, so a bad
    // permutation cannot read out of bounds).
    auto physical = [&](int p, int raw) {
        if constexpr (kIndexedKV) return p < oi_rows ? static_cast<int>(min(static_cast<uint32_t>(raw), sk_last)) : p;
        else return p;
    };
    auto stream_row = [&](int r) {
        const int p = stream_pos(r);
        if constexpr (kIndexedKV) return physical(p, kidx[min(p, oi_rows - 1)]);
        else return p;
    };
    int p2 = 0;  // indexed: this lane's stream position in tile t+2 (its k_index value is in pidx)
    if (prow_owner) {
        prow[0][prow_entry] = stream_row(prow_entry);
        prow[1][prow_entry] = stream_row(kKTile + prow_entry);
    }
    if constexpr (kIndexedKV) {
        p2 = stream_pos(2 * kKTile + prow_entry);
        if (prow_owner) pidx[1][prow_entry] = kidx[min(p2, oi_rows - 1)];
    }

    f32x16 oacc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f, neg_m = 0.0f;
    const float lazy = kLazyLog2 / scale_log2;

    const uint16_t* kh = k + head * sk * D;
    const uint16_t* vh = v + head * sk * D;
    // Per-lane constants of the fragment reads.
    const int arow = lane % 32;                 // S^T A row (key within a 32-key block)
    const int gsub = (lane / 16) % 2;           // 16-lane group parity (V^T channel half)
    const int src = lane % 16;                  // source lane of the transpose read
    // S^T, online softmax and O^T += V^T P^T for NCB consecutive 32-key halves of the tile in
    // (kt, vt), starting at half cb0.
    // after_s() runs once the S^T MFMAs are issued (the next tile's loads go there, so the
    // wait for the load path to accept them overlaps the MFMAs).
    auto compute = [&](auto ncbc, int cb0, const uint16_t* kt, const uint16_t* vt, int base, auto&& after_s)
                       __attribute__((always_inline)) {
        constexpr int NCB = decltype(ncbc)::value;
        const bool partial = base + kKTile > L;
        // S^T for all halves first, so the softmax of one half overlaps MFMAs.
        f32x16 sacc[NCB];
#pragma unroll
        for (int j = 0; j < NCB; ++j) {
            sacc[j] = f32x16{};
            const int krow = 32 * (cb0 + j) + arow;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int pc = (2 * s + h) ^ T::swz_k(krow);
                const u16x8 kf = *reinterpret_cast<const u16x8*>(kt + krow * D + pc * 8);
                sacc[j] = Mfma<DT>::run(kf, qf[s], sacc[j]);
            }
        }
        // K-fragment reads run kLook MFMAs ahead of their use (LDS latency > one MFMA).
        {
            constexpr int kLook = 4;
            __builtin_amdgcn_sched_group_barrier(0x100, kLook, 0);  // DS reads
#pragma unroll
            for (int i = 0; i < NCB * S - kLook; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kLook, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        after_s();
        auto read_vt = [&](int cb, int kk, int nb) __attribute__((always_inline)) {
            s16x4 part[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int vrow = 32 * cb + 16 * kk + 8 * t + 4 * h + src / 4;
                const int d = 32 * nb + 16 * gsub + 4 * (src % 4);
                const int pc = (d / 8) ^ T::swz_v(vrow);
                const uint16_t* a = vt + vrow * D + pc * 8 + (d % 8);
                part[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(a));
            }
            return __builtin_bit_cast(
                u16x8, u32x4{__builtin_bit_cast(u32x2, part[0])[0], __builtin_bit_cast(u32x2, part[0])[1],
                             __builtin_bit_cast(u32x2, part[1])[0], __builtin_bit_cast(u32x2, part[1])[1]});
        };
#pragma unroll
        for (int j = 0; j < NCB; ++j) {
            const int cb = cb0 + j;
            // The V^T fragments of the first 16-key step are read before the softmax, whose
            // VALU work then covers their LDS latency.
            u16x8 vpre[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) vpre[nb] = read_vt(cb, 0, nb);
            __builtin_amdgcn_sched_barrier(0);
            if (partial) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = base + 32 * cb + 8 * (i / 4) + 4 * h + (i % 4);
                    if (key >= L) sacc[j][i] = -INFINITY;
                }
            }
            // Lanes l and l ^ 32 hold the two key halves of one query column and share m_run,
            // so some lane's own maximum passes m_run + lazy exactly when some column's
            // maximum does: the exchange of the halves is needed only to rescale.
            float tmax = sacc[j][0];
#pragma unroll
            for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, sacc[j][i]);
            if (__any(tmax > m_run + lazy)) {
                tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
                const float m_new = fmaxf(m_run, tmax);
                const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
                m_run = m_new;
                neg_m = -m_new * scale_log2;
                l_run *= alpha;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[nb][i] *= alpha;
            }
            uint32_t pp[8];
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][i], scale_log2, neg_m));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][i + 1], scale_log2, neg_m));
                pp[i / 2] = Mfma<DT>::pack2(p0, p1);
                l_run = Mfma<DT>::sum2(pp[i / 2], l_run);
            }
            // O^T += V^T P^T over the two 16-key k-steps of this 32-key half. The V^T
            // fragment (channel 32nb + l%32, 8 keys) comes from two transpose reads: source
            // lane r of each 16-lane group points at key 32cb+16kk+8t+4h+r/4, channels
            // 32nb + 16*gsub + 4*(r%4) .. +3.
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const u16x8 pf = __builtin_bit_cast(u16x8, u32x4{pp[4 * kk], pp[4 * kk + 1], pp[4 * kk + 2],
                                                                pp[4 * kk + 3]});
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const u16x8 af = kk == 0 ? vpre[nb] : read_vt(cb, kk, nb);
                    oacc[nb] = Mfma<DT>::run(af, pf, oacc[nb]);
                }
            }
        }
    };
    if constexpr (kQuantLoad) {
        // The query rows and centroid must arrive before the tile loads below are issued: the
        // compiler does not count those loads, so a later wait for the rows would also wait
        // for the tile.
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
        for (int s = 0; s < S; ++s) asm volatile("" ::"v"(qf[s]), "v"(qc_row[s]));
#endif
    }
    __syncthreads();
    if (ntiles > 0) load_tile_lds<D, kWaves>(ks[0], vs[0], kh, vh, prow[0], wave, lane);
    if constexpr (kQuantLoad) {
        if (qc < qcent_rows) {
            // This lane holds channels 16s + 8h .. +7 of its row and lane l ^ 32 the others:
            // the row's residual bounds are the two lanes' bounds combined. All of it is VALU
            // work on registers that arrived before the first tile's loads were issued, so it
            // runs while those loads are in flight.
            float lo = INFINITY, hi = -INFINITY;
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float r = half_to_f32<DT>(qf[s][i]) - qc_row[s][i];
                    lo = fminf(lo, r);
                    hi = fmaxf(hi, r);
                }
            lo = fminf(lo, __shfl_xor(lo, 32, kWave));
            hi = fmaxf(hi, __shfl_xor(hi, 32, kWave));
            const BaseOffsetRow bo = base_offset_row(lo, hi, levels);
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float c = qc_row[s][i];
                    uint32_t code;
                    const float xh = base_offset_value(half_to_f32<DT>(qf[s][i]) - c, c, bo, code);
                    qf[s][i] = f32_to_half<DT>(xh);
                }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): this wave's tile-0 loads have landed
    __syncthreads();
    auto step = [&](auto bufc, int tile) __attribute__((always_inline)) {
        constexpr int buf = decltype(bufc)::value;
        const bool more = tile + 1 < ntiles;
        // Waves with rows only ever load as one of all kWaves loaders (the other counts mean
        // idle waves carry the loads).
        auto shared_load = [&]() __attribute__((always_inline)) {
            if (more && loaders == kWaves)
                load_tile_lds<D, kWaves>(ks[buf ^ 1], vs[buf ^ 1], kh, vh, prow[buf ^ 1], wave, lane);
        };
        if (wave_active) {
            // Key half hb (with the next tile's loads issued behind its S^T MFMAs), then, for
            // unpaired waves, the other half.
            compute(std::integral_constant<int, 1>{}, hb, ks[buf], vs[buf], tile * kKTile, shared_load);
            if (!split) compute(std::integral_constant<int, 1>{}, 1, ks[buf], vs[buf], tile * kKTile, [] {});
        } else if (more && loader_rank >= 0) {
            if (loaders == kWaves) load_tile_lds<D, kWaves>(ks[buf ^ 1], vs[buf ^ 1], kh, vh, prow[buf ^ 1], wave, lane);
            else if (loaders == 4) load_tile_lds<D, 4>(ks[buf ^ 1], vs[buf ^ 1], kh, vh, prow[buf ^ 1], loader_rank, lane);
            else if (loaders == 2) load_tile_lds<D, 2>(ks[buf ^ 1], vs[buf ^ 1], kh, vh, prow[buf ^ 1], loader_rank, lane);
            else load_tile_lds<D, 1>(ks[buf ^ 1], vs[buf ^ 1], kh, vh, prow[buf ^ 1], loader_rank, lane);
        }
        if constexpr (kIndexedKV) {
            const int p3 = stream_pos((tile + 3) * kKTile + prow_entry);
            if (prow_owner) dma4(kidx + min(p3, oi_rows - 1), lds_addr(&pidx[buf][kRowsPerWave * wave]));
            // Everything but that index load has landed: this wave's tile t+1 loads and the
            // index loaded a tile ago (pidx[buf ^ 1]).
            asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
            if (prow_owner) prow[buf][prow_entry] = physical(p2, pidx[buf ^ 1][prow_entry]);
            p2 = p3;
        } else {
            if (prow_owner) prow[buf][prow_entry] = stream_pos((tile + 2) * kKTile + prow_entry);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's tile t+1 loads
        }
        // The barrier publishes LDS only (prow, the tile t+1 loads, waited for above), so it
        // carries LDS-scoped fences instead of __syncthreads' full ones.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    for (int tile = 0; tile < ntiles; tile += 2) {
        step(std::integral_constant<int, 0>{}, tile);
        if (tile + 1 < ntiles) step(std::integral_constant<int, 1>{}, tile + 1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last index load
    if (split) {
        // Merge the pair's states: the second-half wave (hb = 1) leaves m, l and O in the tile
        // LDS (the K and V buffers, free after the loop's last barrier), the first-half wave
        // rescales both to the larger maximum and adds. Lane l of both waves holds the same
        // query rows. The LDS holds the states of two row blocks at a time, so the H row blocks
        // of an 8-wavefront item take turns in pairs.
#pragma unroll
        for (int r0 = 0; r0 < H; r0 += 2) {
            const bool turn = rb >= r0 && rb < r0 + 2;
            float* xch = reinterpret_cast<float*>(&kvs[0][0]) + ((turn ? rb - r0 : 0) * kWave + lane) * (NB * 16 + 2);
            if (turn && hb == 1 && wave_active) {
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) xch[nb * 16 + i] = oacc[nb][i];
                xch[NB * 16] = m_run;
                xch[NB * 16 + 1] = l_run;
            }
            __syncthreads();
            if (turn && hb == 0 && wave_active) {
                const float m1 = xch[NB * 16], l1 = xch[NB * 16 + 1];
                const float m = fmaxf(m_run, m1);
                // A half without keys has m = -inf (and l = 0, O = 0); both empty leaves O at 0.
                const float a0 = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m_run - m) * scale_log2);
                const float a1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m1 - m) * scale_log2);
                l_run = l_run * a0 + l1 * a1;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[nb][i] = oacc[nb][i] * a0 + xch[nb * 16 + i] * a1;
            }
            if (r0 + 2 < H) __syncthreads();  // the next pair's states overwrite these
        }
        if (hb == 1) return;
    }
    if (!qvalid) return;
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    int64_t orow = q_start + qrow;
    if (out_index && orow < oi_rows) orow = min(static_cast<uint32_t>(out_index[head * oi_rows + orow]), sq_last);
    uint16_t* o = out + (head * sq + orow) * D;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * nb + 8 * g + 4 * h;
            const uint32_t w0 = Mfma<DT>::pack2(oacc[nb][4 * g + 0] * inv, oacc[nb][4 * g + 1] * inv);
            const uint32_t w1 = Mfma<DT>::pack2(oacc[nb][4 * g + 2] * inv, oacc[nb][4 * g + 3] * inv);
            *reinterpret_cast<u32x2*>(o + d0) = u32x2{w0, w1};
        }
}

// Item index g runs on XCD g % 8 in a one-workgroup-per-item grid (workgroups are dispatched
// round-robin over the XCDs), so the band order keeps a head's items on one XCD. The
// persistent form launches only the resident workgroups instead; workgroup w takes the item
// indices g = w % 8 (mod 8) from queue w % 8 with an atomic counter (the same XCD affinity,
// without the dispatcher's in-order round-robin, where a full XCD holds back the workgroups
// behind it) and, when its queue runs dry, from the other queues (the launch's tail then
// spreads over every XCD). Every workgroup leaves when all queues are exhausted (a counter is
// only ever increased, or raised to a band start, so each queue runs out); the last one to
// leave resets the counters for the next call.
// Next non-empty item index from queue `x` onwards (then the other queues), given the first
// candidate k of queue x (already taken with an atomic). Within a band the queue of a head
// (band dividing 8) visits that head's slots in order, so the first empty slot means the rest
// of the band is empty too: the queue is moved past the band at once.
__device__ int resolve_item(int32_t* queues, const int32_t* counts, int cap, int band, int total, int x, int k) {
    const int per_band = band * cap;
    const bool one_head = kItemQueues % band == 0;
    for (int i = 0; i < kItemQueues; ++i) {
        for (;;) {
            const int64_t g = static_cast<int64_t>(k) * kItemQueues + x;
            if (g >= total) break;
            const int gi = static_cast<int>(g);
            const int in_band = gi % per_band;
            const int bh = (gi / per_band) * band + in_band % band;
            if (in_band / band < counts[bh]) return gi;
            if (one_head) {
                // First index of the next band in queue x.
                const int64_t next = (static_cast<int64_t>(gi / per_band) + 1) * per_band;
                const int knext = static_cast<int>((next - x + kItemQueues - 1) / kItemQueues);
                atomicMax(&queues[x], knext);
            }
            k = atomicAdd(&queues[x], 1);
        }
        x = (x + 1) % kItemQueues;
        if (i + 1 < kItemQueues) k = atomicAdd(&queues[x], 1);
    }
    return -1;
}

template <int DT, int D, int kMode, bool kPersist, int kWaves>
__global__ __launch_bounds__(kWaves * kWave, 8 / kWaves) void sparse_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint8_t* __restrict__ selected, const int32_t* __restrict__ kprefix, const int2* __restrict__ segs,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ items, int cap, uint16_t* __restrict__ out,
    const int32_t* __restrict__ out_index, int oi_rows, const int32_t* __restrict__ k_index,
    const float* __restrict__ qcent, int qcent_rows, float levels, int bhn, int band, int sq, int sk, int cq,
    int ck, float scale_log2, int32_t* __restrict__ queues, int nwg) {
    if constexpr (!kPersist) {
        attention_item<DT, D, kMode, kWaves>(blockIdx.x, q, k, v, selected, kprefix, segs, counts, items, cap, out,
                                             out_index, oi_rows, k_index, qcent, qcent_rows, levels, bhn, band, sq,
                                             sk, cq, ck, scale_log2);
    } else {
        __shared__ int next;
        const int total = cap * bhn;
        // An item is taken only when the workgroup is free for it (taking ahead would bind the
        // next item to a workgroup still busy and undo the cost order); the queue of the last
        // item is drained first.
        int x = blockIdx.x % kItemQueues;
        for (;;) {
            if (threadIdx.x == 0) next = resolve_item(queues, counts, cap, band, total, x, atomicAdd(&queues[x], 1));
            __syncthreads();
            const int g = next;
            __syncthreads();  // every wavefront has read `next` before thread 0 writes it again
            if (g < 0) break;
            x = g % kItemQueues;
            attention_item<DT, D, kMode, kWaves>(g, q, k, v, selected, kprefix, segs, counts, items, cap, out,
                                                 out_index, oi_rows, k_index, qcent, qcent_rows, levels, bhn, band, sq,
                                                 sk, cq, ck, scale_log2);
        }
        if (threadIdx.x == 0 && atomicAdd(&queues[kItemQueues], 1) == nwg - 1) {
            for (int x = 0; x <= kItemQueues; ++x)
                __hip_atomic_store(&queues[x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---- Base-Offset scores on the integer MFMA (an extension: the reference runs no such kernel,
// README.md:18) ----
//
// With Base-Offset on, a video query row is q^ = Cq + a + s*u and a video key row
// k^ = Ck + b + t*w (u, w the codes, a, b the row lows, s, t the row scales, Cq, Ck the
// centroids of the row's cluster; peco/quantization.py:13-22 gives this form and the four-term
// expansion). Their dot product is, exactly,
//   q^.k^ = Cq.k^ + a*Sum(k^) + s*(u.Ck + b*Sum(u) + t*(u.w)),
//   Cq.k^ = Cq.Ck + b*Sum(Cq) + t*(Cq.w),   Sum(k^) = Sum(Ck) + D*b + t*Sum(w).
// 8-bit codes are moved to int8 by subtracting 128 (a and b then absorb 128s and 128t).
// - u.w, the only term over query row x key, is exact int32 from v_mfma_i32_32x32x32_i8
//   (half the MFMA issue of the bf16 S^T).
// - u.Ck (query row x key cluster) also runs on the integer MFMA, against the key centroids
//   held as three int8 planes, Ck = cs*(P0 + P1/128 + P2/16384) to within 2^-21 |Ck|max,
//   for 32 kept clusters at a time, into an LDS table per wavefront.
// - Cq.w and Sum(w) are reduced per key from its codes while the tile is staged; Cq.Ck and
//   Sum(Ck) come per tile, Sum(u), a and s per row.
// Scores of video rows against text keys, and every score of a text row (text is not
// quantized, peco/processor.py:141-142), use bf16 MFMA on the fake-quantized rows, as the
// reference computes all of them. The key stream is walked one kept key cluster at a time,
// in tiles of 32 keys (the reference's own tile, peco/kernels/sparse_attention.cu:99-107), so a
// tile has one key centroid. The scores are those of unrounded q^, k^ (the reference rounds
// them to the input dtype before its attention, peco/quantization.py:136).
struct BoAttnArgs {
    const uint16_t* q;         // [bh, sq, D], original token order
    const int32_t* out_index;  // [bh, oi_rows]: cluster-order query row -> original row
    const float* q_cent;       // [bh, kq, D]
    const uint16_t* k;         // [bh, sk, D], cluster order: video rows fake-quantized, text rows raw
    const uint16_t* v;         // [bh, sk, D], cluster order
    const uint8_t* k_codes;    // [bh, oi_rows, D], cluster order
    const float* k_low;        // [bh, oi_rows]
    const float* k_scale;      // [bh, oi_rows]
    const int8_t* kc_planes;   // [bh, kk, 3, D]
    const float* kc_scale;     // [bh, kk]
    const float* kc_sum;       // [bh, kk]: Sum(Ck)
    const float* qk_dot;       // [bh, kk, kq]: Ck.Cq
    const uint8_t* selected;   // [bh, cq, ck]
    const int32_t* kprefix;    // [bh, ck + 1]
    const int32_t* counts;
    const int32_t* items;
    uint16_t* out;
    int cap, oi_rows, kq, kk, bhn, band, sq, sk, cq, ck, shift;
    float levels, scale_log2;
};

constexpr int kBoTile = 32;  // keys per tile

template <int DT, int D>
__global__ __launch_bounds__(256, 2) void bo_attention_kernel(BoAttnArgs A) {
    using T = Tiles<D>;
    constexpr int S = D / 16;          // bf16 k-steps of S^T
    constexpr int S8 = D / 32;         // int8 k-steps
    constexpr int NB = D / 32;         // 32-channel blocks of O^T
    constexpr int CW = D / 16;         // 16-byte code chunks per key row
    constexpr int CH = D / 8;          // 16-byte chunks per 16-bit row
    constexpr int VCH = kBoTile * CH / 256;  // 16-bit row chunks per thread and tile
    constexpr float kLazyLog2 = 8.0f;
    static_assert(VCH >= 1 && kBoTile * CW <= 256, "tile staging assumes 256 threads");
    __shared__ __align__(16) uint16_t kt_lds[2][kBoTile * D];  // codes (D bytes per row) or K rows
    __shared__ __align__(16) uint16_t vt_lds[2][kBoTile * D];
    __shared__ __align__(16) float kq_lds[2][4][kBoTile];      // per key: Cq.k^, Sum(k^), b, t
    __shared__ __align__(16) float gam[4][32][32];             // per wavefront: u.Ck / cs
    __shared__ float tile_cs[2];                                // the tile's cluster scale cs
    __shared__ __align__(16) float cq_lds[D];
    __shared__ int tmp[4];
    extern __shared__ int dyn[];
    const int ck = A.ck;
    int* cl_start = dyn;           // kept, non-empty key clusters of the map row, in order
    int* cl_size = dyn + ck;
    int* cl_kc = dyn + 2 * ck;

    const int per_band = A.band * A.cap;
    const int in_band = blockIdx.x % per_band;
    const int bh = (blockIdx.x / per_band) * A.band + in_band % A.band;
    const int slot = in_band / A.band;
    if (slot >= A.counts[bh]) return;
    const int32_t* item = A.items + (static_cast<int64_t>(bh) * A.cap + slot) * 3;
    const int q_start = item[0], qc = item[1], q_rows = item[2];
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, h = lane / 32;
    const int64_t head = bh;
    const bool video_q = qc < A.kq;
    const uint32_t sq_last = static_cast<uint32_t>(A.sq - 1);

    // Query rows: wavefront w holds rows 32w .. 32w+31 of the item, lane l row l % 32 with
    // channels 16s + 8h .. +7 (the bf16 operand layout).
    const int qrow = wave * 32 + lane % 32;
    const bool qvalid = qrow < q_rows;
    const bool wave_active = wave * 32 < q_rows;
    int64_t qsrc = q_start + qrow;
    if (qvalid && qsrc < A.oi_rows) qsrc = min(static_cast<uint32_t>(A.out_index[head * A.oi_rows + qsrc]), sq_last);
    u16x8 qf[S];
#pragma unroll
    for (int s = 0; s < S; ++s)
        qf[s] = qvalid ? *reinterpret_cast<const u16x8*>(A.q + (head * A.sq + qsrc) * D + 16 * s + 8 * h)
                       : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    f32x8 qcr[S];
    const float* crow = A.q_cent + (head * A.kq + min(qc, A.kq - 1)) * D;
#pragma unroll
    for (int s = 0; s < S; ++s) qcr[s] = video_q ? *reinterpret_cast<const f32x8*>(crow + 16 * s + 8 * h) : f32x8{};
    if (tid < D) cq_lds[tid] = video_q ? crow[tid] : 0.0f;

    // Kept key clusters of this map row with their clamped row ranges, and the tile count.
    int nk, ntiles;
    {
        const uint8_t* sel = A.selected + (head * A.cq + qc) * ck;
        const int32_t* gk = A.kprefix + head * (ck + 1);
        const int per = static_cast<int>(ceil_div(ck, 256));
        const int c0 = tid * per, c1 = min(ck, c0 + per);
        int lcount = 0, ltiles = 0;
        for (int c = c0; c < c1; ++c) {
            const int a = gk[c], e = gk[c + 1];
            if (sel[c] && e > a) {
                ++lcount;
                ltiles += static_cast<int>(ceil_div(e - a, kBoTile));
            }
        }
        int idx = block_scan<4>(lcount, tmp, &nk);
        block_scan<4>(ltiles, tmp, &ntiles);
        for (int c = c0; c < c1; ++c) {
            const int a = gk[c], e = gk[c + 1];
            if (sel[c] && e > a) {
                cl_start[idx] = a;
                cl_size[idx] = e - a;
                cl_kc[idx] = c;
                ++idx;
            }
        }
    }

    // Video rows: Base-Offset quantization at load (base_offset.hpp, the quantizer's own
    // arithmetic): codes u, row low a and scale s, and the fake-quantized row in qf for the
    // bf16 tiles. The int8 operand of k-step s8 holds channels 32 s8 + 16h .. +15: channels
    // 16 sg + 8e .. +7 (sg = 2 s8 + h) come from this lane for e = h and from lane l ^ 32 for
    // e = 1 - h.
    u32x4 u8op[S8];
    float qa = 0.0f, qs = 0.0f, qu = 0.0f, cq_sum = 0.0f;
    if (video_q) {
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float r = half_to_f32<DT>(qf[s][i]) - qcr[s][i];
                lo = fminf(lo, r);
                hi = fmaxf(hi, r);
            }
        lo = fminf(lo, __shfl_xor(lo, 32, kWave));
        hi = fmaxf(hi, __shfl_xor(hi, 32, kWave));
        const BaseOffsetRow bo = base_offset_row(lo, hi, A.levels);
        u32x2 ub[S];
        int usum = 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            ub[s] = u32x2{0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float c = qcr[s][i];
                uint32_t code;
                const float xh = base_offset_value(half_to_f32<DT>(qf[s][i]) - c, c, bo, code);
                qf[s][i] = f32_to_half<DT>(xh);
                usum += static_cast<int>(code);
                ub[s][i / 4] |= ((code - static_cast<uint32_t>(A.shift)) & 0xffu) << (8 * (i % 4));
                cq_sum += c;
            }
        }
#pragma unroll
        for (int s8 = 0; s8 < S8; ++s8) {
            const u32x2 mine = ub[2 * s8 + h];
            const u32x2 send = ub[2 * s8 + 1 - h];
            const u32x2 recv{static_cast<uint32_t>(__shfl_xor(static_cast<int>(send[0]), 32, kWave)),
                             static_cast<uint32_t>(__shfl_xor(static_cast<int>(send[1]), 32, kWave))};
            u8op[s8] = h == 0 ? u32x4{mine[0], mine[1], recv[0], recv[1]} : u32x4{recv[0], recv[1], mine[0], mine[1]};
        }
        qu = static_cast<float>(usum + __shfl_xor(usum, 32, kWave) - A.shift * D);
        cq_sum += __shfl_xor(cq_sum, 32, kWave);
        qs = bo.scale;
        qa = bo.low + static_cast<float>(A.shift) * bo.scale;
    } else {
#pragma unroll
        for (int s8 = 0; s8 < S8; ++s8) u8op[s8] = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();  // the cluster list and cq_lds

    // Tile t covers keys [32 blk, 32 blk + 32) of kept cluster ci. Staging: every thread loads
    // its share of the next tile into registers during the current one and writes it to LDS
    // at the end. 16-bit rows: chunk j of thread t is (row, chunk) of (t + 256 j); code rows:
    // thread t < 32 CW holds row t / CW, chunk t % CW (the CW threads of a row are adjacent).
    const int crow_t = tid / CW, cchunk = tid % CW;
    const bool code_thread = tid < kBoTile * CW;
    u32x4 kreg[VCH], vreg[VCH];  // K rows, or the codes chunk in kreg[0]
    float klow = 0.0f, kscale = 0.0f, ksum_c = 0.0f, qk = 0.0f, kcs = 0.0f;
    const uint32_t xmask = A.shift ? 0x80808080u : 0u;
    auto cluster_of = [&](int ci_, int blk_, int& start, int& nvalid, int& kc, bool& int8) {
        start = cl_start[ci_] + kBoTile * blk_;
        nvalid = min(kBoTile, cl_size[ci_] - kBoTile * blk_);
        kc = cl_kc[ci_];
        int8 = video_q && kc < A.kk;
    };
    auto issue = [&](int ci_, int blk_) __attribute__((always_inline)) {
        int start, nvalid, kc;
        bool int8;
        cluster_of(ci_, blk_, start, nvalid, kc, int8);
#pragma unroll
        for (int j = 0; j < VCH; ++j) {
            const int idx = tid + 256 * j, r = idx / CH, c = idx % CH;
            const int64_t p = start + (r < nvalid ? r : 0);  // rows past the cluster repeat its first
            vreg[j] = *reinterpret_cast<const u32x4*>(A.v + (head * A.sk + p) * D + c * 8);
            if (!int8) kreg[j] = *reinterpret_cast<const u32x4*>(A.k + (head * A.sk + p) * D + c * 8);
        }
        if (int8 && code_thread) {
            const int64_t p = min(start + (crow_t < nvalid ? crow_t : 0), A.oi_rows - 1);
            kreg[0] = *reinterpret_cast<const u32x4*>(A.k_codes + (head * A.oi_rows + p) * D + cchunk * 16);
            if (cchunk == 0) {
                klow = A.k_low[head * A.oi_rows + p];
                kscale = A.k_scale[head * A.oi_rows + p];
                ksum_c = A.kc_sum[head * A.kk + kc];
                qk = A.qk_dot[(head * A.kk + kc) * A.kq + qc];
                kcs = A.kc_scale[head * A.kk + kc];
            }
        }
    };
    auto stage = [&](int buf, int ci_, int blk_) __attribute__((always_inline)) {
        int start, nvalid, kc;
        bool int8;
        cluster_of(ci_, blk_, start, nvalid, kc, int8);
#pragma unroll
        for (int j = 0; j < VCH; ++j) {
            const int idx = tid + 256 * j, r = idx / CH, c = idx % CH;
            *reinterpret_cast<u32x4*>(&vt_lds[buf][r * D + (c ^ T::swz_v(r)) * 8]) = vreg[j];
            if (!int8) *reinterpret_cast<u32x4*>(&kt_lds[buf][r * D + (c ^ T::swz_k(r)) * 8]) = kreg[j];
        }
        if (int8 && code_thread) {
            const u32x4 w = kreg[0] ^ u32x4{xmask, xmask, xmask, xmask};
            uint8_t* kb = reinterpret_cast<uint8_t*>(kt_lds[buf]);
            *reinterpret_cast<u32x4*>(kb + crow_t * D + ((cchunk ^ (crow_t % CW)) * 16)) = w;
            // Sum(w) and Cq.w over this chunk's 16 channels, then over the row's CW chunks.
            int sw = 0;
            float cw = 0.0f;
#pragma unroll
            for (int d4 = 0; d4 < 4; ++d4) {
                const f32x4 cq4 = *reinterpret_cast<const f32x4*>(&cq_lds[cchunk * 16 + 4 * d4]);
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int val = static_cast<int8_t>((w[d4] >> (8 * b)) & 0xffu);
                    sw += val;
                    cw = __builtin_fmaf(static_cast<float>(val), cq4[b], cw);
                }
            }
#pragma unroll
            for (int m = 1; m < CW; m <<= 1) {
                sw += __shfl_xor(sw, m, kWave);
                cw += __shfl_xor(cw, m, kWave);
            }
            if (cchunk == 0) {
                const bool valid = crow_t < nvalid;
                const float t = kscale;
                const float b = klow + static_cast<float>(A.shift) * kscale;
                kq_lds[buf][0][crow_t] = valid ? qk + b * cq_sum + t * cw : 0.0f;
                kq_lds[buf][1][crow_t] = valid ? ksum_c + static_cast<float>(D) * b + t * static_cast<float>(sw) : 0.0f;
                kq_lds[buf][2][crow_t] = valid ? b : 0.0f;
                kq_lds[buf][3][crow_t] = valid ? t : 0.0f;
                if (crow_t == 0) tile_cs[buf] = kcs;
            }
        }
    };

    f32x16 oacc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f, neg_m = 0.0f;
    const float scale_log2 = A.scale_log2;
    const float lazy = kLazyLog2 / scale_log2;
    const int gsub = (lane / 16) % 2, src = lane % 16;

    // u.Ck / cs for the wavefront's rows and kept clusters 32 g .. 32 g + 31 (text clusters and
    // slots past the list give 0, never read): A = the clusters' int8 planes, B = u. One plane
    // at a time keeps the operands' registers few.
    auto gamma_block = [&](int g) __attribute__((always_inline)) {
        const int li = 32 * g + lane % 32;
        const bool ok = li < nk && cl_kc[min(li, nk - 1)] < A.kk;
        const int kcm = ok ? cl_kc[li] : 0;
        const int8_t* pl = A.kc_planes + (head * A.kk + kcm) * 3 * D;
        f32x16 comb{};
#pragma unroll 1
        for (int pn = 0; pn < 3; ++pn) {
            u32x4 pa[S8];
#pragma unroll
            for (int s8 = 0; s8 < S8; ++s8)
                pa[s8] = ok ? *reinterpret_cast<const u32x4*>(pl + pn * D + 32 * s8 + 16 * h) : u32x4{0u, 0u, 0u, 0u};
            i32x16 acc{};
#pragma unroll
            for (int s8 = 0; s8 < S8; ++s8)
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, pa[s8]),
                                                            __builtin_bit_cast(i32x4, u8op[s8]), acc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float wt = pn == 0 ? 1.0f : (pn == 1 ? 1.0f / 128.0f : 1.0f / 16384.0f);
                comb[i] = __builtin_fmaf(static_cast<float>(acc[i]), wt, comb[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) gam[wave][8 * (i / 4) + 4 * h + (i % 4)][lane % 32] = comb[i];
    };

    int ci = 0, blk = 0, gblk = -1;
    if (ntiles > 0) {
        issue(0, 0);
        stage(0, 0, 0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        int start, nvalid, kc;
        bool int8;
        cluster_of(ci, blk, start, nvalid, kc, int8);
        if (int8 && wave_active && ci / 32 != gblk) {
            gblk = ci / 32;
            gamma_block(gblk);
        }
        int nci = ci, nblk = blk + 1;
        if (kBoTile * nblk >= cl_size[ci]) {
            ++nci;
            nblk = 0;
        }
        const bool more = t + 1 < ntiles;
        if (more) issue(nci, nblk);
        if (wave_active) {
            const int row = lane % 32;
            f32x16 sacc;
            if (int8) {
                const uint8_t* kb = reinterpret_cast<const uint8_t*>(kt_lds[buf]);
                i32x16 acc{};
#pragma unroll
                for (int s8 = 0; s8 < S8; ++s8) {
                    const u32x4 af = *reinterpret_cast<const u32x4*>(kb + row * D + (((2 * s8 + h) ^ (row % CW)) * 16));
                    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, af),
                                                                __builtin_bit_cast(i32x4, u8op[s8]), acc, 0, 0, 0);
                }
                const float gm = gam[wave][ci % 32][row] * tile_cs[buf];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int kb0 = 8 * g + 4 * h;
                    const f32x4 bq = *reinterpret_cast<const f32x4*>(&kq_lds[buf][0][kb0]);
                    const f32x4 sk4 = *reinterpret_cast<const f32x4*>(&kq_lds[buf][1][kb0]);
                    const f32x4 bk = *reinterpret_cast<const f32x4*>(&kq_lds[buf][2][kb0]);
                    const f32x4 tk = *reinterpret_cast<const f32x4*>(&kq_lds[buf][3][kb0]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x = __builtin_fmaf(tk[i], static_cast<float>(acc[4 * g + i]),
                                                       __builtin_fmaf(bk[i], qu, gm));
                        sacc[4 * g + i] = __builtin_fmaf(qs, x, __builtin_fmaf(qa, sk4[i], bq[i]));
                    }
                    asm volatile("" ::: "memory");  // keeps each group's per-key reads next to their use
                }
            } else {
                sacc = f32x16{};
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const int pc = (2 * s + h) ^ T::swz_k(row);
                    const u16x8 kf = *reinterpret_cast<const u16x8*>(&kt_lds[buf][row * D + pc * 8]);
                    sacc = Mfma<DT>::run(kf, qf[s], sacc);
                }
            }
            auto read_vt = [&](int kk, int nb) __attribute__((always_inline)) {
                s16x4 part[2];
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int vrow = 16 * kk + 8 * tt + 4 * h + src / 4;
                    const int d = 32 * nb + 16 * gsub + 4 * (src % 4);
                    const int pc = (d / 8) ^ T::swz_v(vrow);
                    const uint16_t* a = &vt_lds[buf][vrow * D + pc * 8 + (d % 8)];
                    part[tt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(a));
                }
                return __builtin_bit_cast(
                    u16x8, u32x4{__builtin_bit_cast(u32x2, part[0])[0], __builtin_bit_cast(u32x2, part[0])[1],
                                 __builtin_bit_cast(u32x2, part[1])[0], __builtin_bit_cast(u32x2, part[1])[1]});
            };
            if (nvalid < kBoTile) {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (8 * (i / 4) + 4 * h + (i % 4) >= nvalid) sacc[i] = -INFINITY;
            }
            float tmax = sacc[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, sacc[i]);
            if (__any(tmax > m_run + lazy)) {
                tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
                const float m_new = fmaxf(m_run, tmax);
                const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * scale_log2);
                m_run = m_new;
                neg_m = -m_new * scale_log2;
                l_run *= alpha;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[nb][i] *= alpha;
            }
            uint32_t pp[8];
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[i], scale_log2, neg_m));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[i + 1], scale_log2, neg_m));
                pp[i / 2] = Mfma<DT>::pack2(p0, p1);
                l_run = Mfma<DT>::sum2(pp[i / 2], l_run);
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const u16x8 pf = __builtin_bit_cast(u16x8, u32x4{pp[4 * kk], pp[4 * kk + 1], pp[4 * kk + 2],
                                                                pp[4 * kk + 3]});
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    oacc[nb] = Mfma<DT>::run(read_vt(kk, nb), pf, oacc[nb]);
                }
            }
        }
        if (more) stage(buf ^ 1, nci, nblk);
        __syncthreads();
        ci = nci;
        blk = nblk;
    }
    if (!qvalid) return;
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    int64_t orow = q_start + qrow;
    if (orow < A.oi_rows) orow = min(static_cast<uint32_t>(A.out_index[head * A.oi_rows + orow]), sq_last);
    uint16_t* o = A.out + (head * A.sq + orow) * D;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * nb + 8 * g + 4 * h;
            const uint32_t w0 = Mfma<DT>::pack2(oacc[nb][4 * g + 0] * inv, oacc[nb][4 * g + 1] * inv);
            const uint32_t w1 = Mfma<DT>::pack2(oacc[nb][4 * g + 2] * inv, oacc[nb][4 * g + 3] * inv);
            *reinterpret_cast<u32x2*>(o + d0) = u32x2{w0, w1};
        }
}

size_t build_lds_bytes(int cq, int ck) {
    const int cap = kSortCap;
    return sizeof(int) * ((static_cast<size_t>(ck) + 2 * cq + 2) & ~static_cast<size_t>(1)) + sizeof(uint64_t) * cap;
}

}  // namespace
}  // namespace peco

using namespace peco;

// Work-list footprint in int32 elements; always <= the reference's
// BH*(CK+2+3*(ceil(SQ/16)+CQ)) (peco/attention_cuda.py:112-113).
PECO_API size_t peco_sparse_attention_workspace_size(int bh, int sq, int sk, int cq, int ck) {
    (void)sk;
    if (bh < 1 || sq < 0 || cq < 1 || ck < 1) return 0;
    return static_cast<size_t>(bh) + static_cast<size_t>(bh) * (ck + 1) +
           static_cast<size_t>(bh) * item_capacity(sq, cq) * 3;
}

namespace peco {
namespace {

// Heads whose items run together (the grid is slot-major within a band, and workgroup b runs
// on XCD b % 8). Every item of a head streams its K/V rows:
// - when one head's K/V fits an XCD's 4 MB L2 and bh is a multiple of 8, bands of 8 heads put
//   one head on each XCD at a time, so its items stream from that L2 (480p: 3.6 MB per head;
//   3.7% faster than one band of all 24 heads, which gives each XCD three heads at a time);
// - else, when all heads' K/V fit in kAllHeadsBytes, one band of all heads;
// - else the largest divisor of bh up to kMaxBand whose K/V fit in the 256 MB MALL (of bands
//   of 1, 2, 4 and all 24 heads, 4 ran fastest at both 32896 and 119056 tokens).
constexpr double kL2Bytes = 4.0 * 1024 * 1024;
constexpr int kXcds = 8;
constexpr double kAllHeadsBytes = 96.0 * 1024 * 1024;
constexpr double kMallBytes = 256.0 * 1024 * 1024;
constexpr int kMaxBand = 4;
int attention_head_band(int bh, int sk, int d) {
    const double kv = 4.0 * static_cast<double>(sk) * d;  // K and V bytes of one head (16-bit)
    if (kv <= kL2Bytes && bh % kXcds == 0) return kXcds;
    if (bh * kv <= kAllHeadsBytes) return bh;
    for (int band = std::min(bh, kMaxBand); band > 1; --band)
        if (bh % band == 0 && band * kv <= kMallBytes) return band;
    return 1;
}

// Launch of the attention kernel over a built work list (map + kprefix, or segs).
// q_centroids (nullable, with out_index) selects the kQuantQ input mode, or kIndexedQuantQ
// with k_index.
// queues (nullable): the work list's item queue counters. Given, and with at least
// kPersistItems item slots per resident workgroup, the grid is the persistent one of
// sparse_attention_kernel (two resident workgroups per CU take items from the queues): 544p
// attention 5.4% and 720p 4.2% faster than one workgroup per item, while at 480p (5.6 slots
// per workgroup, items of about 100 us) taking each item costs more than it saves (+2.3%).
constexpr int kPersistItems = 8;
int launch_attention_kernel(const void* q, const void* k, const void* v, const uint8_t* selected,
                            const int32_t* kprefix, const int2* segs, const int32_t* counts, const int32_t* items,
                            int cap, void* output, const int32_t* out_index, int out_index_rows,
                            const int32_t* k_index, const float* q_centroids, int q_clusters, int bits, int bh,
                            int sq, int sk, int d, int cq, int ck, int dtype, int32_t* queues, hipStream_t s) {
    const int mode = k_index ? (q_centroids ? kIndexedQuantQ : kIndexed) : (q_centroids ? kQuantQ : kPacked);
    const float levels = static_cast<float>((1 << bits) - 1);
    const size_t lds_attn = sizeof(int) * 2 * (static_cast<size_t>(ck) + 1);
    const float scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(d)));
    const int64_t total = static_cast<int64_t>(cap) * bh;
    // Items of 2 * kQTile rows (attention_item_rows, the builders' rule) run on 8-wavefront
    // workgroups, one per CU; others on 4-wavefront ones, two per CU.
    const int waves = attention_item_rows(sq) == 2 * kQTile ? 8 : 4;
    const int nwg = static_cast<int>(
        std::min<int64_t>(total, (8 / waves) * static_cast<int64_t>(device_compute_units())));
    if (queues && total < static_cast<int64_t>(kPersistItems) * nwg) queues = nullptr;
    const dim3 grid(static_cast<unsigned>(queues ? nwg : total));
    const int band = attention_head_band(bh, sk, d);
    const auto* qp = static_cast<const uint16_t*>(q);
    const auto* kp = static_cast<const uint16_t*>(k);
    const auto* vp = static_cast<const uint16_t*>(v);
    auto* op = static_cast<uint16_t*>(output);
#define PECO_ATTN_P(DT_, D_, M_, P_, W_)                                                                           \
    hipLaunchKernelGGL((sparse_attention_kernel<DT_, D_, M_, P_, W_>), grid, dim3(W_ * kWave), lds_attn, s, qp, kp, \
                       vp, selected, kprefix, segs, counts, items, cap, op, out_index, out_index_rows, k_index,      \
                       q_centroids, q_clusters, levels, bh, band, sq, sk, cq, ck, scale_log2, queues, nwg)
#define PECO_ATTN(DT_, D_, M_, W_)                                                                                 \
    do {                                                                                                           \
        if (queues) PECO_ATTN_P(DT_, D_, M_, true, W_);                                                            \
        else PECO_ATTN_P(DT_, D_, M_, false, W_);                                                                  \
    } while (0)
#define PECO_ATTN_W(DT_, D_, M_)                                                                                   \
    do {                                                                                                           \
        if (waves == 8) PECO_ATTN(DT_, D_, M_, 8);                                                                 \
        else PECO_ATTN(DT_, D_, M_, 4);                                                                            \
    } while (0)
#define PECO_ATTN_D(DT_, M_)                                                                                       \
    do {                                                                                                           \
        if (d == 128) PECO_ATTN_W(DT_, 128, M_);                                                                   \
        else PECO_ATTN_W(DT_, 64, M_);                                                                             \
    } while (0)
#define PECO_ATTN_M(DT_)                                                                                           \
    do {                                                                                                           \
        if (mode == kIndexed) PECO_ATTN_D(DT_, kIndexed);                                                          \
        else if (mode == kQuantQ) PECO_ATTN_D(DT_, kQuantQ);                                                       \
        else if (mode == kIndexedQuantQ) PECO_ATTN_D(DT_, kIndexedQuantQ);                                         \
        else PECO_ATTN_D(DT_, kPacked);                                                                            \
    } while (0)
    if (dtype == kBF16) PECO_ATTN_M(kBF16);
    else PECO_ATTN_M(kF16);
#undef PECO_ATTN_M
#undef PECO_ATTN_D
#undef PECO_ATTN_W
#undef PECO_ATTN
#undef PECO_ATTN_P
    return hipGetLastError();
}

// Shared launcher: k_index (nullable) selects the indexed-input kernel (inputs in original
// token order, read through out_index for Q and k_index for K/V).
int launch_sparse_attention(const void* q, const void* k, const void* v, const uint8_t* selected,
                            const int* q_sizes, const int* k_sizes, void* output, const int32_t* out_index,
                            int out_index_rows, const int32_t* k_index, const int32_t* kept_keys, int* workspace,
                            size_t workspace_ints,
                            int bh, int sq, int sk, int d, int cq, int ck, int dtype, void* stream) {
    if (!q || !k || !v || !selected || !q_sizes || !k_sizes || !output || !workspace || bh < 1 || bh > 65535 ||
        sq < 0 || sk < 0 || cq < 1 || ck < 1 || (d != 64 && d != 128) || (dtype != kF16 && dtype != kBF16) ||
        (out_index && (out_index_rows < 0 || out_index_rows > sq)) ||
        (k_index && (!out_index || out_index_rows > sk)))
        return kInvalidValue;
    if (sq == 0) return kOk;
    if (workspace_ints < peco_sparse_attention_workspace_size(bh, sq, sk, cq, ck)) return kWorkspaceTooSmall;
    const size_t lds_build = build_lds_bytes(cq, ck);
    const size_t lds_attn = sizeof(int) * 2 * (static_cast<size_t>(ck) + 1);
    if (lds_build > 60 * 1024 || lds_attn > 24 * 1024) return kUnsupportedShape;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (kept_keys)
        hipLaunchKernelGGL(build_work_kernel<true>, dim3(bh), dim3(256), lds_build, s, selected, q_sizes, k_sizes,
                           kept_keys, workspace, bh, sq, sk, cq, ck, attention_item_rows(sq));
    else
        hipLaunchKernelGGL(build_work_kernel<false>, dim3(bh), dim3(256), lds_build, s, selected, q_sizes, k_sizes,
                           nullptr, workspace, bh, sq, sk, cq, ck, attention_item_rows(sq));
    const WorkLayout W = work_layout(workspace, bh, sq, cq, ck);
    return launch_attention_kernel(q, k, v, selected, W.kprefix, nullptr, W.counts, W.items, W.cap, output, out_index,
                                   out_index_rows, k_index, nullptr, 0, 0, bh, sq, sk, d, cq, ck, dtype, nullptr, s);
}

}  // namespace
}  // namespace peco

// Extended entry: out_index (nullable, int32 [bh, out_index_rows]) scatters output row
// j < out_index_rows of head b to row out_index[b, j] (rows past out_index_rows keep their
// position), fusing the inverse permutation into the epilogue.
PECO_API int peco_sparse_attention_ex(const void* q, const void* k, const void* v, const uint8_t* selected,
                                      const int* q_sizes, const int* k_sizes, void* output, const int32_t* out_index,
                                      int out_index_rows, const int32_t* kept_keys, int* workspace,
                                      size_t workspace_ints, int bh, int sq, int sk, int d, int cq, int ck, int dtype,
                                      void* stream) {
    return launch_sparse_attention(q, k, v, selected, q_sizes, k_sizes, output, out_index, out_index_rows, nullptr,
                                   kept_keys, workspace, workspace_ints, bh, sq, sk, d, cq, ck, dtype, stream);
}

// Gathering entry: q, k, v (and output) stay in original token order. The first index_rows
// rows of each head are read in cluster order through q_index (queries, also the output
// scatter) and k_index (keys and values), so no packed copies are needed. kept_keys (nullable,
// [bh, cq]) gives each query cluster's kept key rows, as the selection launch writes them;
// the work-list builder then orders items without reading the map.
PECO_API int peco_sparse_attention_indexed(const void* q, const void* k, const void* v, const uint8_t* selected,
                                           const int* q_sizes, const int* k_sizes, void* output,
                                           const int32_t* q_index, const int32_t* k_index, int index_rows,
                                           const int32_t* kept_keys, int* workspace, size_t workspace_ints, int bh,
                                           int sq, int sk, int d, int cq, int ck, int dtype, void* stream) {
    if (index_rows < 0 || (index_rows > 0 && (!q_index || !k_index))) return kInvalidValue;
    if (index_rows == 0) q_index = k_index = nullptr;  // nothing is permuted
    return launch_sparse_attention(q, k, v, selected, q_sizes, k_sizes, output, q_index, index_rows, k_index, kept_keys,
                                   workspace, workspace_ints, bh, sq, sk, d, cq, ck, dtype, stream);
}

// Work-list entry: the work list and kept-segment lists come from peco_select_work (same
// bh, sq and map dims cq x ck), so no builder runs and no map row is read. Q/K/V addressing
// and out_index/k_index are those of peco_sparse_attention_ex (k_index null) and
// peco_sparse_attention_indexed (out_index = q_index, k_index given). With q_centroids
// (fp32 [bh, q_clusters, d]; needs out_index) Q is in original order: query row
// j < out_index_rows is read from row out_index[j] and Base-Offset fake-quantized with `bits`
// against its cluster's centroid as it is loaded; K and V are then in cluster order, or in
// original order read through k_index when it is given. The work buffer is written: the
// persistent grid takes items with atomic counters in it (left zero at the end), so two
// launches sharing one work buffer must not overlap.
PECO_API int peco_sparse_attention_work(const void* q, const void* k, const void* v, void* output,
                                        const int32_t* out_index, int out_index_rows, const int32_t* k_index,
                                        const float* q_centroids, int q_clusters, int bits, int32_t* work,
                                        size_t work_ints, int bh, int sq, int sk, int d, int cq, int ck, int dtype,
                                        void* stream) {
    if (!q || !k || !v || !output || !work || bh < 1 || bh > 65535 || sq < 0 || sk < 0 || cq < 1 || ck < 1 ||
        (d != 64 && d != 128) || (dtype != kF16 && dtype != kBF16) ||
        (out_index && (out_index_rows < 0 || out_index_rows > sq)) || (k_index && (!out_index || out_index_rows > sk)) ||
        (q_centroids && (!out_index || q_clusters < 1 || q_clusters > cq || (bits != 4 && bits != 8))))
        return kInvalidValue;
    if (sq == 0) return kOk;
    if (work_ints < sel_work_ints(bh, sq, cq, ck)) return kWorkspaceTooSmall;
    if (sizeof(int) * 2 * (static_cast<size_t>(ck) + 1) > 24 * 1024) return kUnsupportedShape;
    const SelWork W = sel_work_layout(work, bh, sq, cq, ck);
    return launch_attention_kernel(q, k, v, nullptr, nullptr, W.segs, W.counts, W.items, W.cap, output, out_index,
                                   out_index_rows, k_index, q_centroids, q_centroids ? q_clusters : 0,
                                   q_centroids ? bits : 0, bh, sq, sk, d, cq, ck, dtype, W.queues,
                                   static_cast<hipStream_t>(stream));
}

// Base-Offset integer-score attention (an extension with no counterpart in the reference; see
// bo_attention_kernel). Map-driven like peco_sparse_attention_ex (selected, q_sizes, k_sizes
// as there, extended with the text partition), with Q in original token order (video row
// j < oi_rows of the cluster order read from row out_index[j], which also places the output)
// and K, V, the key codes, lows and scales in cluster order, as peco_kmeans_fit_pack writes
// them. q_centroids [bh, kq, d] and the key centroid planes (kc_planes int8 [bh, kk, 3, d],
// kc_scale, kc_sum fp32 [bh, kk], qk_dot fp32 [bh, kk, kq] = Ck.Cq) describe the first kq
// query and kk key clusters of the map (the video ones); bits is the codes' width (4 or 8).
PECO_API int peco_base_offset_attention(const void* q, const int32_t* out_index, const float* q_centroids, int kq,
                                        const void* k, const void* v, const uint8_t* k_codes, const float* k_low,
                                        const float* k_scale, const int8_t* kc_planes, const float* kc_scale,
                                        const float* kc_sum, const float* qk_dot, int kk, int bits,
                                        const uint8_t* selected, const int* q_sizes, const int* k_sizes,
                                        void* output, int* workspace, size_t workspace_ints, int bh, int sq, int sk,
                                        int oi_rows, int d, int cq, int ck, int dtype, void* stream) {
    if (!q || !out_index || !q_centroids || !k || !v || !k_codes || !k_low || !k_scale || !kc_planes || !kc_scale ||
        !kc_sum || !qk_dot || !selected || !q_sizes || !k_sizes || !output || !workspace || bh < 1 || bh > 65535 ||
        sq < 1 || sk < 1 || cq < 1 || ck < 1 || kq < 1 || kq > cq || kk < 1 || kk > ck || oi_rows < 1 ||
        oi_rows > sq || oi_rows > sk || (d != 64 && d != 128) || (dtype != kF16 && dtype != kBF16) ||
        (bits != 4 && bits != 8))
        return kInvalidValue;
    if (workspace_ints < peco_sparse_attention_workspace_size(bh, sq, sk, cq, ck)) return kWorkspaceTooSmall;
    const size_t lds_build = build_lds_bytes(cq, ck);
    const size_t lds_list = sizeof(int) * 3 * static_cast<size_t>(ck);
    if (lds_build > 60 * 1024 || lds_list > 24 * 1024) return kUnsupportedShape;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // The integer-score kernel runs 4-wavefront workgroups: items of kQTile rows.
    hipLaunchKernelGGL(build_work_kernel<false>, dim3(bh), dim3(256), lds_build, s, selected, q_sizes, k_sizes, nullptr,
                       workspace, bh, sq, sk, cq, ck, kQTile);
    const WorkLayout W = work_layout(workspace, bh, sq, cq, ck);
    BoAttnArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.out_index = out_index;
    a.q_cent = q_centroids;
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.k_codes = k_codes;
    a.k_low = k_low;
    a.k_scale = k_scale;
    a.kc_planes = kc_planes;
    a.kc_scale = kc_scale;
    a.kc_sum = kc_sum;
    a.qk_dot = qk_dot;
    a.selected = selected;
    a.kprefix = W.kprefix;
    a.counts = W.counts;
    a.items = W.items;
    a.out = static_cast<uint16_t*>(output);
    a.cap = W.cap;
    a.oi_rows = oi_rows;
    a.kq = kq;
    a.kk = kk;
    a.bhn = bh;
    a.band = attention_head_band(bh, sk, d);
    a.sq = sq;
    a.sk = sk;
    a.cq = cq;
    a.ck = ck;
    a.shift = bits == 8 ? 128 : 0;
    a.levels = static_cast<float>((1 << bits) - 1);
    a.scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(d)));
    const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(W.cap) * bh));
#define PECO_BO(DT_, D_) hipLaunchKernelGGL((bo_attention_kernel<DT_, D_>), grid, dim3(256), lds_list, s, a)
    if (dtype == kBF16) {
        if (d == 128) PECO_BO(kBF16, 128);
        else PECO_BO(kBF16, 64);
    } else {
        if (d == 128) PECO_BO(kF16, 128);
        else PECO_BO(kF16, 64);
    }
#undef PECO_BO
    return hipGetLastError();
}

// Reference ABI (peco/kernels/sparse_attention.cu:210): workspace holds
// BH*(CK+2+3*(ceil(SQ/16)+CQ)) int32, as sized by the reference's Python wrapper.
PECO_API int peco_sparse_attention(const void* q, const void* k, const void* v, const uint8_t* selected,
                                   const int* q_sizes, const int* k_sizes, void* output, int* workspace, int bh,
                                   int sq, int sk, int d, int cq, int ck, int dtype, void* stream) {
    if (bh < 1 || sq < 0) return kInvalidValue;
    const size_t ref_ints = static_cast<size_t>(bh) * (ck + 2 + 3 * (ceil_div(sq, 16) + cq));
    return peco_sparse_attention_ex(q, k, v, selected, q_sizes, k_sizes, output, nullptr, 0, nullptr, workspace,
                                    ref_ints, bh, sq, sk, d, cq, ck, dtype, stream);
}

// ---- Allocation-free variant (no counterpart in the reference) ----
//
// The work list lives in a file-scope device array instead of a caller workspace, for callers
// that cannot allocate (code under HIP graph capture, serving loops that forbid allocation).
// Each GPU holds its own copy of the array (4 MiB) until the process ends. Every call on a
// GPU uses that GPU's copy, so calls that overlap on one GPU (two streams, or two host
// threads) race; calls on one stream are ordered. The builder writes every entry it later
// reads, so nothing needs clearing between calls.
namespace peco {
namespace {

constexpr size_t kStaticWorkInts = size_t(1) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) int32_t scratch[kStaticWorkInts];

std::mutex g_scratch_mutex;
int32_t* g_scratch[kMaxDevices] = {};

// Device address of the current device's `scratch`, looked up once per device. The host-side
// name `scratch` is only a stand-in for the symbol and is never passed to a kernel.
int current_scratch(int32_t** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return kInvalidValue;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch[dev] = static_cast<int32_t*>(ptr);
    }
    *out = g_scratch[dev];
    return kOk;
}

}  // namespace
}  // namespace peco

PECO_API int peco_sparse_attention_noalloc(const void* q, const void* k, const void* v, const uint8_t* selected,
                                           const int* q_sizes, const int* k_sizes, void* output, int bh, int sq,
                                           int sk, int d, int cq, int ck, int dtype, void* stream) {
    if (bh < 1 || sq < 0 || cq < 1 || ck < 1) return kInvalidValue;
    if (peco_sparse_attention_workspace_size(bh, sq, sk, cq, ck) > kStaticWorkInts) return kScratchExceeded;
    int32_t* work = nullptr;
    const int e = current_scratch(&work);
    if (e != kOk) return e;
    return launch_sparse_attention(q, k, v, selected, q_sizes, k_sizes, output, nullptr, 0, nullptr, nullptr, work,
                                   kStaticWorkInts, bh, sq, sk, d, cq, ck, dtype, stream);
}
