/*
 * C-ABI of libpeco_hip.so: the PECO per-layer attention hot path on MI355X (gfx950).
 *
 * Conventions (same as the reference's two CUDA libraries):
 *   - every pointer is device memory owned by the caller, unless stated otherwise;
 *   - every call is asynchronous on `stream` (a hipStream_t; torch's current stream);
 *   - return 0 on success, a hipError_t value on a runtime error, 1 (hipErrorInvalidValue)
 *     on bad arguments, or a PECO status >= 20001 (see peco_cluster_error_message).
 * dtype codes: 0 = fp16, 1 = bf16, 2 = fp32.
 */
#ifndef PECO_HIP_H
#define PECO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Reference ABI: peco/kernels/kmeans.cu (bound by peco/clustering_cuda.py:65-71) ---- */

/* Replaces peco_assign_tokens_to_centers, peco/kernels/kmeans.cu:139.
 * labels[b,t] = argmin_j fma(-2, x_t.c_j, |c_j|^2), lowest j on ties (fixed-order fp32).
 * center_norms [batch, clusters] receives |c_j|^2; when it is null the first batch*clusters
 * floats of scratch hold them (one of the two must be given). chunk_size is unused.
 * Allocates nothing. */
int peco_assign_tokens_to_centers(const float* x, const float* centers, int32_t* labels, float* scratch,
                                  float* center_norms, int batch, int tokens, int dims, int clusters,
                                  int chunk_size, void* stream);

/* Replaces peco_recompute_cluster_centers, peco/kernels/kmeans.cu:179.
 * sums (nullable) / counts / means of x rows per label; sums accumulate in token order;
 * an empty cluster keeps `previous`. */
int peco_recompute_cluster_centers(const float* x, const int32_t* labels, const float* previous, float* sums,
                                   int32_t* counts, float* means, int batch, int tokens, int dims, int clusters,
                                   void* stream);

/* Replaces peco_reorder_token_features, peco/kernels/kmeans.cu:200.
 * inverse=0: out[b,j] = in[b, indices[b,j]]; inverse=1: out[b, indices[b,j]] = in[b,j].
 * item_size 2 or 4 (bit copy of fp16/bf16/fp32 rows). */
int peco_reorder_token_features(const void* input, const int32_t* indices, void* output, int batch_heads,
                                int tokens, int dims, int item_size, int inverse, void* stream);

/* Replaces peco_cluster_error_message, peco/kernels/kmeans.cu:220. Static string. */
const char* peco_cluster_error_message(int code);

/* ---- Reference ABI: peco/kernels/sparse_attention.cu (bound by peco/attention_cuda.py:57-60) ---- */

/* Replaces peco_sparse_attention, peco/kernels/sparse_attention.cu:210.
 * q [bh,sq,d], k/v [bh,sk,d] (fp16/bf16, d in {64,128}), selected bool [bh,cq,ck],
 * int32 sizes [bh,cq]/[bh,ck]; workspace holds bh*(ck+2+3*(ceil(sq/16)+cq)) int32
 * (the reference's own size). Fully masked rows are zero. */
int peco_sparse_attention(const void* q, const void* k, const void* v, const uint8_t* selected,
                          const int* q_sizes, const int* k_sizes, void* output, int* workspace, int bh, int sq,
                          int sk, int d, int cq, int ck, int dtype, void* stream);

/* Replaces peco_attention_error_string, peco/kernels/sparse_attention.cu:232. */
const char* peco_attention_error_string(int code);

/* ---- Extensions (no counterpart in the reference's native code) ---- */

/* ABI revision of this library. */
int peco_abi_version(void);

/* Stable argsort of labels per batch entry as a counting sort (replaces the torch.argsort
 * of peco/clustering.py:105). indices[b,j] = original token at sorted position j;
 * ranks (nullable) = inverse permutation; counts (nullable) [b,clusters];
 * offsets (nullable) [b,clusters+1]. clusters <= 16384. */
size_t peco_cluster_sort_workspace_size(int batch, int tokens, int clusters);
int peco_cluster_sort(const int32_t* labels, int batch, int tokens, int clusters, int32_t* indices, int32_t* ranks,
                      int32_t* counts, int32_t* offsets, void* workspace, size_t workspace_bytes, void* stream);

/* Fused Lloyd fit (peco/clustering.py:17-89 with tol=0) of num_problems (1 or 2)
 * independent problems. The problems' batch entries run as four chains of launches, three of
 * them on library-owned streams of the current device, forked from `stream` and joined back to
 * it with events, so the call is ordered on `stream` like a single chain. Problem i: x[i] rows [batch, tokens, dims]
 * in `dtype` with batch stride x_batch_stride[i] elements (NULL or 0 = tokens*dims),
 * initial centres centers_in[i] fp32 [batch, clusters, dims]; outputs centers_out[i],
 * labels[i] [batch,tokens], counts[i] [batch,clusters], sorted_indices[i] (stable sort
 * of the final labels) and offsets[i] [batch, clusters+1]. dims in {64, 128}. */
size_t peco_kmeans_workspace_size(int batch, int tokens, int clusters, int dims);
int peco_kmeans_fit(int num_problems, const void* const* x, const int64_t* x_batch_stride,
                    const float* const* centers_in, float* const* centers_out, int32_t* const* labels,
                    int32_t* const* counts, int32_t* const* sorted_indices, int32_t* const* offsets,
                    const int* batch, const int* tokens, const int* clusters, int dims, int dtype, int iterations,
                    void* workspace, size_t workspace_bytes, void* stream);

/* peco_kmeans_fit that also packs (fuses peco/processor.py:141-149 into the fit): for
 * problem i with hat[i] non-null, hat[i] [batch, length, dims] receives x's rows
 * Base-Offset fake-quantized with bits[i] (4 or 8) against the final centres, in the final
 * cluster order (hat_order 0, written by the last update) or each at its own token position
 * (hat_order 1, written by one token-parallel launch after the last update), then x's rows
 * [tokens, length) unchanged (the text; x_batch_stride[i] must cover length rows);
 * with_in[i] -> with_out[i] ([batch, length, dims], both or neither, hat_order 0 only) are
 * gathered in the same order with their text rows copied. codes[i], low[i], scale[i] (all
 * three or none; uint8 [batch, tokens, dims], fp32 [batch, tokens]) receive the Base-Offset
 * payload of hat[i]'s first tokens rows in the same order, as quantize_base_offset computes
 * it (peco/quantization.py:97-128). Labels, centres, counts and the permutation are those of
 * peco_kmeans_fit. (ABI revision 4: codes/low/scale added; revision 5: hat_order.) */
int peco_kmeans_fit_pack(int num_problems, const void* const* x, const int64_t* x_batch_stride,
                         const float* const* centers_in, float* const* centers_out, int32_t* const* labels,
                         int32_t* const* counts, int32_t* const* sorted_indices, int32_t* const* offsets,
                         const int* batch, const int* tokens, const int* clusters, int dims, int dtype, int iterations,
                         void* const* hat, const int* bits, const void* const* with_in, void* const* with_out,
                         uint8_t* const* codes, float* const* low, float* const* scale, int length, int hat_order,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Diagnostic of the certified assignment (no counterpart in the reference): for bf16 x
 * [batch, tokens, dims] and fp32 centres, screened[b,t,j] receives the MFMA screen value
 * |c_j|^2 - 2 x_t.c_j (split-bf16 centres) that the assignment compares, labels the certified
 * labels, center_norms the canonical norms. peco_kmeans_screen_bound gives the coefficients
 * kappa (of |x||c|) and gamma (of |c|^2) of the error bound the certification assumes. */
int peco_kmeans_screen(const void* x, int dtype, const float* centers, float* center_norms, int32_t* labels,
                       float* screened, int batch, int tokens, int dims, int clusters, void* stream);
void peco_kmeans_screen_bound(int dims, float* kappa, float* gamma);

/* Base-Offset PE quantizer (peco/quantization.py:97-150), dims in {64, 128}.
 * encode: codes uint8 [batch,tokens,dims] (nullable), low/scale fp32 [batch,tokens] (nullable).
 * decode: x_hat in `dtype` from codes/low/scale. fake_quant: encode+decode in one pass. */
int peco_base_offset_encode(const void* x, int dtype, const int32_t* labels, const float* centroids, int batch,
                            int tokens, int clusters, int dims, int bits, uint8_t* codes, float* low, float* scale,
                            void* stream);
int peco_base_offset_decode(const uint8_t* codes, const float* low, const float* scale, const int32_t* labels,
                            const float* centroids, int batch, int tokens, int clusters, int dims, int dtype,
                            void* out, void* stream);
int peco_base_offset_fake_quant(const void* x, int dtype, const int32_t* labels, const float* centroids, int batch,
                                int tokens, int clusters, int dims, int bits, void* out, void* stream);

/* One launch packing up to 3 tensors [batch, length, dims] (fuses peco/processor.py:141-149):
 * rows [0, video) in the order of indices[i] [batch, video], fake-quantized against
 * labels[i]/centroids[i] when bits[i] is 4 or 8; rows [video, length) copied unchanged. */
int peco_pack_clustered(const void* const* inputs, void* const* outputs, const int32_t* const* indices,
                        const int32_t* const* labels, const float* const* centroids, const int* clusters,
                        const int* bits, int num_tensors, int batch, int length, int video, int dims, int dtype,
                        void* stream);

/* peco_sparse_attention with an explicit workspace size (int32 elements, at least
 * peco_sparse_attention_workspace_size) and an optional out_index [bh, out_index_rows]:
 * output row j < out_index_rows of head b is written to row out_index[b,j]; later rows keep
 * their position (fuses peco/clustering.py:128-136 and the text rows of processor.py:153-156).
 * kept_keys (nullable, int32 [bh, cq]) gives the key rows each query cluster keeps, as
 * peco_select_cluster_connections writes them; it only orders the work items and spares the
 * work-list builder its pass over the map. (ABI revision 2 added kept_keys.) */
size_t peco_sparse_attention_workspace_size(int bh, int sq, int sk, int cq, int ck);
int peco_sparse_attention_ex(const void* q, const void* k, const void* v, const uint8_t* selected,
                             const int* q_sizes, const int* k_sizes, void* output, const int32_t* out_index,
                             int out_index_rows, const int32_t* kept_keys, int* workspace, size_t workspace_ints,
                             int bh, int sq, int sk, int d, int cq, int ck, int dtype, void* stream);

/* peco_sparse_attention_ex on Q/K/V in their original token order: stream row j <
 * index_rows of head b reads query row q_index[b,j] and key/value row k_index[b,j], and output
 * row j is written to row q_index[b,j]; later rows (text) keep their position. Fuses the
 * gather of peco/clustering.py:112-125 (processor.py:143-149) and the restore of
 * clustering.py:128-136 (processor.py:153-156) into the attention launch. index_rows <= min(sq, sk).
 * kept_keys (nullable) [bh, cq]: key rows kept by each query cluster, as
 * peco_select_cluster_connections writes them; they only order the work items. */
int peco_sparse_attention_indexed(const void* q, const void* k, const void* v, const uint8_t* selected,
                                  const int* q_sizes, const int* k_sizes, void* output, const int32_t* q_index,
                                  const int32_t* k_index, int index_rows, const int32_t* kept_keys, int* workspace,
                                  size_t workspace_ints, int bh, int sq, int sk, int d, int cq, int ck, int dtype,
                                  void* stream);

/* Cluster-pair selection (replaces the torch ops of peco/clustering.py:140-186), one
 * wavefront per query-cluster row: count-weighted softmax of centroid scores, stable
 * descending order, keep while the preceding mass is < p (all when p == 1), at least
 * max(1, minimum) pairs, empty clusters never pair. qc [bh,cq,dims], kc [bh,ck,dims] fp32,
 * counts int32. With extend != 0 the map is [bh,cq+2,ck+2] with the valid-text/padding
 * groups of peco/processor.py:68-84 and ext_q/ext_k receive the extended sizes. kept_keys
 * (nullable) [bh, cq(+2)] receives the number of key rows each map row keeps (the cost of
 * its query rows for the attention work list). Shapes: ck <= 2048 and dims <= 256 with
 * 4*(8*dims + 64*(dims+1)) + 8*ck bytes of LDS at most 64 KiB (dims 128 takes any ck);
 * larger ones return 20002. */
int peco_select_cluster_connections(const float* qc, const float* kc, const int32_t* q_counts,
                                    const int32_t* k_counts, int bh, int cq, int ck, int dims, float p, int minimum,
                                    int extend, int valid_text, int text, uint8_t* map, int32_t* ext_q,
                                    int32_t* ext_k, int32_t* kept_keys, void* stream);

/* ABI revision 3 added peco_select_work_size, peco_select_work, peco_sparse_attention_work
 * and peco_kmeans_fit_pack. */

/* ABI revision 4 added peco_base_offset_attention and the codes/low/scale outputs of
 * peco_kmeans_fit_pack. */

/* ABI revision 5 added the hat_order argument of peco_kmeans_fit_pack, q_centroids together
 * with k_index in peco_sparse_attention_work, and made its work buffer writable. */

/* int32 elements of peco_select_work's work buffer (bh entries, sq query rows, a cq(+2) x
 * ck(+2) map). */
size_t peco_select_work_size(int bh, int sq, int cq, int ck, int extend);

/* The selection of peco_select_cluster_connections fused with the attention's work list
 * (replaces select_cluster_connections, peco/clustering.py:155-186, extend_text_partition,
 * peco/processor.py:68-84, and the reference's per-launch work map,
 * peco/kernels/sparse_attention.cu:17-46, whose kernel scans every map row's flags, :94-96).
 * One launch writes, per map row, the kept-segment list of its key stream (kept clusters with
 * rows, adjacent ones merged, each as {first physical row - stream offset, stream offset}) and
 * its stream length, and, per entry, the attention items in cost order (the entry's last
 * workgroup to finish orders them). map, ext_q and ext_k are optional here. The first bh
 * int32 of work (8-byte aligned) are arrival counters, and 16 int32 after the items are the
 * attention's item queue counters: both zero before the first call on a buffer (allocate it
 * zeroed), and every selection (arrival counters) and attention (queue counters) call leaves
 * them zero, so one buffer serves calls ordered on a stream but not overlapping calls. sq and
 * sk are the attention's query and key lengths (video + text). An item holds at most 128
 * query rows, 256 when sq is 65536 or more (the attention then runs 8-wavefront workgroups);
 * the rule depends on sq alone, which the attention call must repeat. */
int peco_select_work(const float* qc, const float* kc, const int32_t* q_counts, const int32_t* k_counts, int bh,
                     int cq, int ck, int dims, float p, int minimum, int extend, int valid_text, int text, int sq,
                     int sk, uint8_t* map, int32_t* ext_q, int32_t* ext_k, int32_t* work, size_t work_ints,
                     void* stream);

/* Sparse attention over the work list of peco_select_work (same bh and sq; cq, ck are the
 * map's dimensions, text groups included): no builder launch and no map read (replaces
 * peco/kernels/sparse_attention.cu:210 with the work list precomputed). out_index and
 * k_index as in peco_sparse_attention_ex (k_index null: q/k/v in cluster order) and
 * peco_sparse_attention_indexed (out_index = q_index: q/k/v in original order). With
 * q_centroids (fp32 [bh, q_clusters, d], out_index given) q is in original order: query row
 * j < out_index_rows is read from row out_index[j] and Base-Offset fake-quantized with `bits`
 * (4 or 8) against the centroid of its cluster as it is loaded (peco/processor.py:141 and the
 * Q gather fused into the kernel; the text rows' clusters, q_clusters and up, are not
 * quantized); k and v are then in cluster order (k_index null) or in original order read
 * through k_index. The work buffer is written: the persistent grid's item queue counters live
 * in it (every launch leaves them zero), so launches sharing one buffer must not overlap. */
int peco_sparse_attention_work(const void* q, const void* k, const void* v, void* output, const int32_t* out_index,
                               int out_index_rows, const int32_t* k_index, const float* q_centroids, int q_clusters,
                               int bits, int32_t* work, size_t work_ints, int bh, int sq, int sk, int d, int cq,
                               int ck, int dtype, void* stream);

/* Cluster-sparse attention with Base-Offset scores on the integer MFMA. No counterpart in the
 * reference, which reconstructs Q/K and runs floating-point attention (peco/quantization.py:
 * 1-22 gives the four-term expansion it leaves unused; README.md:18). Map-driven like
 * peco_sparse_attention_ex (selected, q_sizes, k_sizes of the map extended with the text
 * partition, workspace of peco_sparse_attention_workspace_size). q is in original token order:
 * video row j < oi_rows of the cluster order is read from row out_index[j] (which also places
 * its output row) and Base-Offset quantized with `bits` (4 or 8) against q_centroids [bh, kq,
 * d]. k (video rows fake-quantized), v, k_codes uint8 [bh, oi_rows, d], k_low and k_scale fp32
 * [bh, oi_rows] are in key cluster order, as peco_kmeans_fit_pack writes them. The key
 * centroids enter as three int8 planes kc_planes [bh, kk, 3, d] with kc_scale [bh, kk]
 * (centroid = kc_scale * (P0 + P1/128 + P2/16384)), their sums kc_sum [bh, kk] and
 * qk_dot [bh, kk, kq] = Ck.Cq. Video x video scores are the exact expansion of
 * (Cq + a + s u).(Ck + b + t w) with u.w from v_mfma_i32_32x32x32_i8; scores involving text
 * rows use the fake-quantized rows on bf16/fp16 MFMA, as the reference does. */
int peco_base_offset_attention(const void* q, const int32_t* out_index, const float* q_centroids, int kq,
                               const void* k, const void* v, const uint8_t* k_codes, const float* k_low,
                               const float* k_scale, const int8_t* kc_planes, const float* kc_scale,
                               const float* kc_sum, const float* qk_dot, int kk, int bits, const uint8_t* selected,
                               const int* q_sizes, const int* k_sizes, void* output, int* workspace,
                               size_t workspace_ints, int bh, int sq, int sk, int oi_rows, int d, int cq, int ck,
                               int dtype, void* stream);

/* peco_sparse_attention without a workspace argument. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc). The work list lives in a static per-device array of 1048576 int32
 * (4 MiB per GPU, held until the process ends); a problem whose work list
 * (peco_sparse_attention_workspace_size) is larger returns 20004. Calls that overlap on one
 * GPU share that array and race; calls ordered on one stream do not. Allocates nothing. */
int peco_sparse_attention_noalloc(const void* q, const void* k, const void* v, const uint8_t* selected,
                                  const int* q_sizes, const int* k_sizes, void* output, int bh, int sq, int sk,
                                  int d, int cq, int ck, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PECO_HIP_H */
