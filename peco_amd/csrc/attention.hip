// Stage 4: cluster-sparse flash attention on MFMA (gfx950), with its device work list.
//
// Semantics (peco/attention_cuda.py:75-83, peco/kernels/sparse_attention.cu:17-46,94,135-158,187):
//   out_i = sum_{j : map[cq(i), ck(j)]} softmax_j(q_i.k_j / sqrt(D)) v_j, and 0 when row i
//   keeps no key. Query and key rows are grouped by cluster in the order of q_sizes/k_sizes.
//
// Work list (one 256-thread workgroup per (batch*head)):
//   cluster offsets are min(S, prefix of max(0, size)) (the reference's clamped running sum),
//   each query cluster is cut into items of <= 128 rows, and the items of one head are
//   ordered by descending cost rows * kept_keys. The attention grid is slot-major
//   (block = slot * BH + bh): the costliest item of every head starts first, and with BH a
//   multiple of 8 all items of one head land on one XCD, whose L2 then holds that head's K/V.
//
// Attention workgroup = one item: 4 waves x 32 query rows. The kept key clusters of the
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
#include "common.hpp"

#include <algorithm>

namespace peco {
namespace {

constexpr int kQTile = 128;   // query rows per item (4 waves x 32)
constexpr int kKTile = 64;    // keys per LDS tile
constexpr int kSortCap = 2048;

struct WorkLayout {
    int32_t* counts;   // [bh]
    int32_t* kprefix;  // [bh, ck + 1]
    int32_t* items;    // [bh, cap, 3]: q_start, q_cluster, q_rows
    int cap;
};

__host__ __device__ inline int item_capacity(int sq, int cq) {
    return static_cast<int>(ceil_div(sq, kQTile)) + min(cq, sq);
}

__host__ __device__ inline WorkLayout work_layout(int32_t* ws, int bh, int sq, int cq, int ck) {
    WorkLayout w;
    w.cap = item_capacity(sq, cq);
    w.counts = ws;
    w.kprefix = ws + bh;
    w.items = w.kprefix + static_cast<int64_t>(bh) * (ck + 1);
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

// Exclusive scan over a 256-thread block (sum of all values in *total).
__device__ __forceinline__ int block_scan256(int v, int* tmp, int* total) {
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int inc = wave_incl_scan(v);
    __syncthreads();
    if (lane == kWave - 1) tmp[wave] = inc;
    __syncthreads();
    int base = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        base += w < wave ? tmp[w] : 0;
        sum += tmp[w];
    }
    *total = sum;
    return base + inc - v;
}

__global__ __launch_bounds__(256) void build_work_kernel(const uint8_t* __restrict__ selected,
                                                         const int* __restrict__ q_sizes,
                                                         const int* __restrict__ k_sizes, int32_t* ws, int bhn,
                                                         int sq, int sk, int cq, int ck) {
    extern __shared__ int lds[];
    __shared__ int tmp[4];
    const int bh = blockIdx.x;
    WorkLayout W = work_layout(ws, bhn, sq, cq, ck);
    int* ksz = lds;              // [ck] clamped key cluster sizes
    int* qoff = ksz + ck;        // [cq + 1] clamped query offsets
    int* kept = qoff + cq + 1;   // [cq] kept keys per query cluster
    uint64_t* keys = reinterpret_cast<uint64_t*>(lds + ((ck + 2 * cq + 1 + 1) & ~1));  // [pow2 >= cap] sort keys
    int32_t* kpre = W.kprefix + static_cast<int64_t>(bh) * (ck + 1);
    // Key cluster offsets: min(sk, prefix of max(0, size)).
    {
        const int per = static_cast<int>(ceil_div(ck, 256));
        const int c0 = threadIdx.x * per, c1 = min(ck, c0 + per);
        int local = 0;
        for (int c = c0; c < c1; ++c) local += max(0, k_sizes[static_cast<int64_t>(bh) * ck + c]);
        int total;
        int run = block_scan256(local, tmp, &total);
        for (int c = c0; c < c1; ++c) {
            const int a = min(sk, run);
            run += max(0, k_sizes[static_cast<int64_t>(bh) * ck + c]);
            const int e = min(sk, run);
            kpre[c] = a;
            ksz[c] = e - a;
        }
        if (threadIdx.x == 0) kpre[ck] = min(sk, total);
    }
    // Query cluster offsets.
    {
        const int per = static_cast<int>(ceil_div(cq, 256));
        const int c0 = threadIdx.x * per, c1 = min(cq, c0 + per);
        int local = 0;
        for (int c = c0; c < c1; ++c) local += max(0, q_sizes[static_cast<int64_t>(bh) * cq + c]);
        int total;
        int run = block_scan256(local, tmp, &total);
        for (int c = c0; c < c1; ++c) {
            qoff[c] = min(sq, run);
            run += max(0, q_sizes[static_cast<int64_t>(bh) * cq + c]);
        }
        if (threadIdx.x == 0) qoff[cq] = min(sq, total);
    }
    __syncthreads();
    // Kept keys per query cluster (one wave per query cluster, lanes over key clusters).
    {
        const int wave = threadIdx.x / kWave, lane = lane_id();
        for (int c = wave; c < cq; c += 4) {
            const uint8_t* row = selected + (static_cast<int64_t>(bh) * cq + c) * ck;
            int s = 0;
            for (int kc = lane; kc < ck; kc += kWave) s += row[kc] ? ksz[kc] : 0;
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) s += __shfl_xor(s, m, kWave);
            if (lane == 0) kept[c] = s;
        }
    }
    __syncthreads();
    // Items per query cluster.
    const int per = static_cast<int>(ceil_div(cq, 256));
    const int c0 = threadIdx.x * per, c1 = min(cq, c0 + per);
    int local = 0;
    for (int c = c0; c < c1; ++c) local += static_cast<int>(ceil_div(qoff[c + 1] - qoff[c], kQTile));
    int count;
    int slot = block_scan256(local, tmp, &count);
    int32_t* items = W.items + static_cast<int64_t>(bh) * W.cap * 3;
    const bool sortable = count <= kSortCap;
    for (int c = c0; c < c1; ++c) {
        const int rows = qoff[c + 1] - qoff[c];
        for (int r = 0; r < rows; r += kQTile, ++slot) {
            const int n = min(kQTile, rows - r);
            if (sortable) {
                const uint32_t cost = static_cast<uint32_t>(min<int64_t>(static_cast<int64_t>(n) * kept[c], 0x7fffffff));
                // Pack (descending cost, item payload index) for an ascending sort.
                keys[slot] = (static_cast<uint64_t>(~cost) << 32) | static_cast<uint32_t>(slot);
            }
            items[3 * slot + 0] = qoff[c] + r;
            items[3 * slot + 1] = c;
            items[3 * slot + 2] = n;
        }
    }
    if (threadIdx.x == 0) W.counts[bh] = count;
    if (!sortable || count <= 1) return;
    int n2 = 1;
    while (n2 < count) n2 <<= 1;
    for (int i = count + threadIdx.x; i < n2; i += 256) keys[i] = ~0ull;
    __syncthreads();
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n2; i += 256) {
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
    // Permute items into cost order (read all, then write all).
    int v[3 * 8];
    int nmine = 0;
    for (int i = threadIdx.x; i < count && nmine < 8; i += 256, ++nmine) {
        const int src = static_cast<int>(keys[i] & 0xffffffffu);
        v[3 * nmine + 0] = items[3 * src + 0];
        v[3 * nmine + 1] = items[3 * src + 1];
        v[3 * nmine + 2] = items[3 * src + 2];
    }
    __syncthreads();
    nmine = 0;
    for (int i = threadIdx.x; i < count && nmine < 8; i += 256, ++nmine) {
        items[3 * i + 0] = v[3 * nmine + 0];
        items[3 * i + 1] = v[3 * nmine + 1];
        items[3 * i + 2] = v[3 * nmine + 2];
    }
}

template <int DT> struct Mfma;
template <> struct Mfma<kBF16> {
    static __device__ __forceinline__ f32x16 run(u16x8 a, u16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    }
};
template <> struct Mfma<kF16> {
    static __device__ __forceinline__ f32x16 run(u16x8 a, u16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
};

// LDS strides (in 16-bit elements): K tile rows of D channels (+8 pad), V^T rows of 64 keys (+4 pad).
template <int D> struct Tiles {
    static constexpr int kRow = D + 8;
    static constexpr int vRow = kKTile + 4;
    static constexpr int kElems = kKTile * kRow;
    static constexpr int vElems = D * vRow;
};

template <int DT, int D>
__global__ __launch_bounds__(256, 2) void sparse_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint8_t* __restrict__ selected, const int32_t* __restrict__ ws, uint16_t* __restrict__ out,
    const int32_t* __restrict__ out_index, int bhn, int sq, int sk, int cq, int ck, float scale_log2) {
    using T = Tiles<D>;
    constexpr int S = D / 16;       // k-steps of S^T over channels
    constexpr int NB = D / 32;      // 32-channel blocks of O^T
    __shared__ uint16_t ks[T::kElems];
    __shared__ uint16_t vt[T::vElems];
    __shared__ int prow[kKTile];
    __shared__ int tmp[4];
    extern __shared__ int dyn[];
    int* soff = dyn;            // [ck] stream offset of each key cluster
    int* kpre = dyn + ck;       // [ck + 1]

    const int bh = blockIdx.x % bhn;
    const int slot = blockIdx.x / bhn;
    const WorkLayout W = work_layout(const_cast<int32_t*>(ws), bhn, sq, cq, ck);
    if (slot >= W.counts[bh]) return;
    const int32_t* item = W.items + (static_cast<int64_t>(bh) * W.cap + slot) * 3;
    const int q_start = item[0], qc = item[1], q_rows = item[2];
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, h = lane / 32;

    // Key stream of this query cluster.
    const uint8_t* sel = selected + (static_cast<int64_t>(bh) * cq + qc) * ck;
    const int32_t* gk = W.kprefix + static_cast<int64_t>(bh) * (ck + 1);
    int L;
    {
        const int per = static_cast<int>(ceil_div(ck, 256));
        const int c0 = tid * per, c1 = min(ck, c0 + per);
        int local = 0;
        for (int c = c0; c < c1; ++c) {
            const int a = gk[c], e = gk[c + 1];
            kpre[c] = a;
            local += sel[c] ? e - a : 0;
        }
        if (tid == 0) kpre[ck] = gk[ck];
        int run = block_scan256(local, tmp, &L);
        for (int c = c0; c < c1; ++c) {
            soff[c] = run;
            run += sel[c] ? gk[c + 1] - gk[c] : 0;
        }
    }

    // Q^T operand: lane holds query row (32*wave + l%32), channels 16s + 8h .. +7.
    const int qrow = wave * 32 + (lane % 32);
    const bool qvalid = qrow < q_rows;
    const bool wave_active = wave * 32 < q_rows;
    const int64_t head = static_cast<int64_t>(bh);
    u16x8 qf[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        qf[s] = qvalid ? *reinterpret_cast<const u16x8*>(q + (head * sq + q_start + qrow) * D + 16 * s + 8 * h)
                       : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    f32x16 oacc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) oacc[nb] = f32x16{};
    float m_run = -INFINITY, l_run = 0.0f;

    const uint16_t* kh = k + head * sk * D;
    const uint16_t* vh = v + head * sk * D;
    const int ntiles = static_cast<int>(ceil_div(L, kKTile));
    for (int tile = 0; tile < ntiles; ++tile) {
        const int base = tile * kKTile;
        __syncthreads();  // previous tile fully consumed; soff/kpre visible
        if (tid < kKTile) {
            const int r = base + tid;
            int phys = -1;
            if (r < L) {
                // Largest cluster c with soff[c] <= r (it is non-empty and holds r).
                int lo = 0, hi = ck - 1;
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (soff[mid] <= r) lo = mid;
                    else hi = mid - 1;
                }
                phys = kpre[lo] + (r - soff[lo]);
            }
            prow[tid] = phys;
        }
        __syncthreads();
        // K tile: row-major [key][D] (+pad). 16 lanes per key row, 16 bytes each.
        {
            constexpr int CH = D / 8;          // 16-byte chunks per row
            constexpr int RPP = 256 / CH;      // rows per pass
#pragma unroll
            for (int pass = 0; pass < kKTile / RPP; ++pass) {
                const int kr = pass * RPP + tid / CH;
                const int ch = tid % CH;
                const int pr = prow[kr];
                u32x4 val = u32x4{0, 0, 0, 0};
                if (pr >= 0) val = *reinterpret_cast<const u32x4*>(kh + static_cast<int64_t>(pr) * D + ch * 8);
                *reinterpret_cast<u32x4*>(ks + kr * T::kRow + ch * 8) = val;
            }
        }
        // V^T tile: [D][64 keys] (+pad). Thread: 4 consecutive keys x 8 channels.
        {
            constexpr int DC = D / 8;
            for (int id = tid; id < 16 * DC; id += 256) {
                const int kq = id % 16, dc = id / 16;
                u16x8 rows[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int pr = prow[4 * kq + r];
                    rows[r] = pr >= 0 ? *reinterpret_cast<const u16x8*>(vh + static_cast<int64_t>(pr) * D + dc * 8)
                                      : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t lo = rows[0][i] | (static_cast<uint32_t>(rows[1][i]) << 16);
                    const uint32_t hi = rows[2][i] | (static_cast<uint32_t>(rows[3][i]) << 16);
                    *reinterpret_cast<u32x2*>(vt + (dc * 8 + i) * T::vRow + 4 * kq) = u32x2{lo, hi};
                }
            }
        }
        __syncthreads();
        if (!wave_active) continue;

        // S^T for two 32-key blocks.
        f32x16 sacc[2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            f32x16 acc = {};
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const u16x8 kf = *reinterpret_cast<const u16x8*>(ks + (32 * cb + lane % 32) * T::kRow + 16 * s + 8 * h);
                acc = Mfma<DT>::run(kf, qf[s], acc);
            }
            sacc[cb] = acc;
        }
        // Online softmax (per query l%32; the two lane halves hold disjoint keys).
        float tmax = -INFINITY;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = base + 32 * cb + 8 * (i / 4) + 4 * h + (i % 4);
                const float sv = key < L ? sacc[cb][i] * scale_log2 : -INFINITY;
                sacc[cb][i] = sv;
                tmax = fmaxf(tmax, sv);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
        const float m_new = fmaxf(m_run, tmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        m_run = m_new;
        float psum = 0.0f;
        u16x8 pf[4];  // P^T operands for the four 16-key k-steps
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float pv = __builtin_amdgcn_exp2f(sacc[cb][i] - m_use);
                psum += pv;
                // k-step ks = 2*cb + (i/8); element j = i % 8 (keys 8g+4h+r, g = i/4).
                pf[2 * cb + i / 8][i % 8] = f32_to_half<DT>(pv);
            }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[nb][i] *= alpha;
        // O^T += V^T P^T.
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const uint16_t* vrow = vt + (32 * nb + lane % 32) * T::vRow;
#pragma unroll
            for (int kstep = 0; kstep < 4; ++kstep) {
                const u32x2 a0 = *reinterpret_cast<const u32x2*>(vrow + 16 * kstep + 4 * h);
                const u32x2 a1 = *reinterpret_cast<const u32x2*>(vrow + 16 * kstep + 8 + 4 * h);
                const u32x4 af = u32x4{a0[0], a0[1], a1[0], a1[1]};
                oacc[nb] = Mfma<DT>::run(__builtin_bit_cast(u16x8, af), pf[kstep], oacc[nb]);
            }
        }
    }
    if (!qvalid) return;
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    int64_t orow = q_start + qrow;
    if (out_index) orow = out_index[head * sq + orow];
    uint16_t* o = out + (head * sq + orow) * D;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * nb + 8 * g + 4 * h;
            const uint32_t w0 = f32_to_half<DT>(oacc[nb][4 * g + 0] * inv) |
                                (static_cast<uint32_t>(f32_to_half<DT>(oacc[nb][4 * g + 1] * inv)) << 16);
            const uint32_t w1 = f32_to_half<DT>(oacc[nb][4 * g + 2] * inv) |
                                (static_cast<uint32_t>(f32_to_half<DT>(oacc[nb][4 * g + 3] * inv)) << 16);
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

// Extended entry: out_index (nullable, int32 [bh, sq]) scatters output row j of head b to
// row out_index[b, j], fusing the inverse permutation into the epilogue.
PECO_API int peco_sparse_attention_ex(const void* q, const void* k, const void* v, const uint8_t* selected,
                                      const int* q_sizes, const int* k_sizes, void* output, const int32_t* out_index,
                                      int* workspace, size_t workspace_ints, int bh, int sq, int sk, int d, int cq,
                                      int ck, int dtype, void* stream) {
    if (!q || !k || !v || !selected || !q_sizes || !k_sizes || !output || !workspace || bh < 1 || bh > 65535 ||
        sq < 0 || sk < 0 || cq < 1 || ck < 1 || (d != 64 && d != 128) || (dtype != kF16 && dtype != kBF16))
        return kInvalidValue;
    if (sq == 0) return kOk;
    if (workspace_ints < peco_sparse_attention_workspace_size(bh, sq, sk, cq, ck)) return kWorkspaceTooSmall;
    const size_t lds_build = build_lds_bytes(cq, ck);
    const size_t lds_attn = sizeof(int) * (2 * static_cast<size_t>(ck) + 1);
    if (lds_build > 60 * 1024 || lds_attn > 24 * 1024) return kUnsupportedShape;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(build_work_kernel, dim3(bh), dim3(256), lds_build, s, selected, q_sizes, k_sizes, workspace, bh,
                       sq, sk, cq, ck);
    const int cap = item_capacity(sq, cq);
    const float scale_log2 = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(d)));
    const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(cap) * bh));
    const auto* qp = static_cast<const uint16_t*>(q);
    const auto* kp = static_cast<const uint16_t*>(k);
    const auto* vp = static_cast<const uint16_t*>(v);
    auto* op = static_cast<uint16_t*>(output);
#define PECO_ATTN(DT_, D_)                                                                                        \
    hipLaunchKernelGGL((sparse_attention_kernel<DT_, D_>), grid, dim3(256), lds_attn, s, qp, kp, vp, selected,    \
                       workspace, op, out_index, bh, sq, sk, cq, ck, scale_log2)
    if (dtype == kBF16) {
        if (d == 128) PECO_ATTN(kBF16, 128);
        else PECO_ATTN(kBF16, 64);
    } else {
        if (d == 128) PECO_ATTN(kF16, 128);
        else PECO_ATTN(kF16, 64);
    }
#undef PECO_ATTN
    return hipGetLastError();
}

// Reference ABI (peco/kernels/sparse_attention.cu:210): workspace holds
// BH*(CK+2+3*(ceil(SQ/16)+CQ)) int32, as sized by the reference's Python wrapper.
PECO_API int peco_sparse_attention(const void* q, const void* k, const void* v, const uint8_t* selected,
                                   const int* q_sizes, const int* k_sizes, void* output, int* workspace, int bh,
                                   int sq, int sk, int d, int cq, int ck, int dtype, void* stream) {
    if (bh < 1 || sq < 0) return kInvalidValue;
    const size_t ref_ints = static_cast<size_t>(bh) * (ck + 2 + 3 * (ceil_div(sq, 16) + cq));
    return peco_sparse_attention_ex(q, k, v, selected, q_sizes, k_sizes, output, nullptr, workspace, ref_ints, bh, sq,
                                    sk, d, cq, ck, dtype, stream);
}
