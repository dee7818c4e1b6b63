/*
 * CPU oracle for the PECO per-layer attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is compiled into oracle/_build/libpeco_oracle.so
 * and is loaded by tests/ and __graft_entry__.smoke(), which check the GPU results against
 * it, and by bench.py's cpu_baseline leg, which times it as the CPU baseline. The product
 * library (peco_amd) never links or calls it.
 *
 * Every function restates the reference algorithm with a fixed, documented fp32
 * operation order, so that the HIP kernels can be required to match it bit for bit:
 *
 *   oracle_center_norms   n_j = sum_d fl(c_jd * c_jd), d ascending, no FMA
 *                         (reference: centers.square().sum(-1), peco/clustering.py:67)
 *   oracle_assign         D_j = fma(-2, dot_j, n_j), dot_j = fma chain over d ascending,
 *                         label = argmin_j D_j, lowest j on ties
 *                         (peco/clustering.py:68-73; tie rule peco/kernels/kmeans.cu:43,55-56)
 *   oracle_update         sums in token order (fp32 adds), mean = sum / count,
 *                         empty cluster keeps previous centre
 *                         (peco/clustering.py:74-80)
 *   oracle_kmeans_fit     Lloyd loop with explicit initial centres, fixed iterations
 *                         (peco/clustering.py:45-89 with tol=0)
 *   oracle_stable_sort    stable argsort of labels, plus cluster offsets
 *                         (peco/clustering.py:92-108)
 *   oracle_base_offset    min-max centroid-residual quantizer and its decode
 *                         (peco/quantization.py:97-136)
 *   oracle_sparse_attention  cluster-masked softmax(QK^T/sqrt(D))V in double precision,
 *                         completely masked rows return zero
 *                         (peco/attention_cuda.py:75-83; peco/kernels/sparse_attention.cu:17-46,94,187)
 *
 * Build: gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp -shared -fPIC (oracle/build.py).
 * -ffp-contract=off keeps every a*b+c that is not written as fmaf() as two roundings.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* n_j = sum_d fl(c_jd^2), sequential in d, separate multiply and add. */
void oracle_center_norms(const float* centers, int batch, int clusters, int dims, float* norms) {
    for (int64_t j = 0; j < (int64_t)batch * clusters; ++j) {
        const float* c = centers + j * dims;
        float s = 0.0f;
        for (int d = 0; d < dims; ++d) {
            float sq = c[d] * c[d];
            s = s + sq;
        }
        norms[j] = s;
    }
}

/* Canonical distances of one token to all clusters of one batch entry.
 * ct is the transposed centre block [dims][clusters]; every (token, cluster) pair is a
 * sequential fmaf chain over d ascending (vectorised across clusters, not across d). */
static void token_distances(const float* x, const float* ct, const float* norms, int clusters,
                            int dims, float* acc, float* dist) {
    for (int j = 0; j < clusters; ++j) acc[j] = 0.0f;
    for (int d = 0; d < dims; ++d) {
        const float xv = x[d];
        const float* row = ct + (int64_t)d * clusters;
        for (int j = 0; j < clusters; ++j) acc[j] = fmaf(xv, row[j], acc[j]);
    }
    for (int j = 0; j < clusters; ++j) dist[j] = fmaf(-2.0f, acc[j], norms[j]);
}

static void transpose_block(const float* c, int clusters, int dims, float* ct) {
    for (int j = 0; j < clusters; ++j)
        for (int d = 0; d < dims; ++d) ct[(int64_t)d * clusters + j] = c[(int64_t)j * dims + d];
}

/* labels[b,t] = argmin_j D_j (lowest j on ties). best/second (nullable) receive the smallest
 * and second-smallest canonical distance of every token, for near-tie certification. */
void oracle_assign(const float* x, const float* centers, const float* norms, int batch, int tokens,
                   int dims, int clusters, int32_t* labels, float* best, float* second) {
#pragma omp parallel
    {
        float* ct = (float*)malloc(sizeof(float) * (size_t)clusters * dims);
        float* acc = (float*)malloc(sizeof(float) * (size_t)clusters);
        float* dist = (float*)malloc(sizeof(float) * (size_t)clusters);
        for (int b = 0; b < batch; ++b) {
            transpose_block(centers + (int64_t)b * clusters * dims, clusters, dims, ct);
#pragma omp for schedule(static)
            for (int t = 0; t < tokens; ++t) {
                const int64_t row = (int64_t)b * tokens + t;
                token_distances(x + row * dims, ct, norms + (int64_t)b * clusters, clusters, dims, acc, dist);
                int arg = 0;
                float m1 = dist[0], m2 = INFINITY;
                for (int j = 1; j < clusters; ++j) {
                    if (dist[j] < m1) { m2 = m1; m1 = dist[j]; arg = j; }
                    else if (dist[j] < m2) { m2 = dist[j]; }
                }
                labels[row] = arg;
                if (best) best[row] = m1;
                if (second) second[row] = m2;
            }
        }
        free(ct); free(acc); free(dist);
    }
}

/* sums/counts/means from labels; sums are accumulated in token order with fp32 adds. */
void oracle_update(const float* x, const int32_t* labels, const float* previous, int batch, int tokens,
                   int dims, int clusters, float* sums, int32_t* counts, float* means) {
#pragma omp parallel for schedule(static)
    for (int b = 0; b < batch; ++b) {
        float* s = sums + (int64_t)b * clusters * dims;
        int32_t* cnt = counts + (int64_t)b * clusters;
        memset(s, 0, sizeof(float) * (size_t)clusters * dims);
        memset(cnt, 0, sizeof(int32_t) * (size_t)clusters);
        for (int t = 0; t < tokens; ++t) {
            const int64_t row = (int64_t)b * tokens + t;
            const int c = labels[row];
            float* dst = s + (int64_t)c * dims;
            const float* src = x + row * dims;
            for (int d = 0; d < dims; ++d) dst[d] = dst[d] + src[d];
            cnt[c] += 1;
        }
        for (int c = 0; c < clusters; ++c) {
            const int64_t base = ((int64_t)b * clusters + c) * dims;
            for (int d = 0; d < dims; ++d)
                means[base + d] = cnt[c] > 0 ? sums[base + d] / (float)cnt[c] : previous[base + d];
        }
    }
}

/* Stable argsort by label. indices[b, j] = original token at sorted position j;
 * offsets[b, c] = first sorted position of cluster c, offsets[b, clusters] = tokens. */
void oracle_stable_sort(const int32_t* labels, int batch, int tokens, int clusters, int32_t* indices,
                        int32_t* offsets) {
    for (int b = 0; b < batch; ++b) {
        const int32_t* lab = labels + (int64_t)b * tokens;
        int32_t* off = offsets + (int64_t)b * (clusters + 1);
        int32_t* idx = indices + (int64_t)b * tokens;
        memset(off, 0, sizeof(int32_t) * (size_t)(clusters + 1));
        for (int t = 0; t < tokens; ++t) off[lab[t] + 1] += 1;
        for (int c = 0; c < clusters; ++c) off[c + 1] += off[c];
        int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)clusters);
        memcpy(cursor, off, sizeof(int32_t) * (size_t)clusters);
        for (int t = 0; t < tokens; ++t) idx[cursor[lab[t]]++] = t;
        free(cursor);
    }
}

/* Lloyd's k-means with explicit initial centres and a fixed iteration count.
 * centers_out receives the means of the returned partition (empty clusters keep their
 * previous centre); indices/offsets (nullable) receive the stable sort of the final labels. */
void oracle_kmeans_fit(const float* x, const float* init, int batch, int tokens, int dims, int clusters,
                       int iterations, int32_t* labels, float* centers_out, int32_t* counts,
                       int32_t* indices, int32_t* offsets) {
    const size_t csize = (size_t)batch * clusters * dims;
    float* centers = (float*)malloc(sizeof(float) * csize);
    float* means = (float*)malloc(sizeof(float) * csize);
    float* sums = (float*)malloc(sizeof(float) * csize);
    float* norms = (float*)malloc(sizeof(float) * (size_t)batch * clusters);
    memcpy(centers, init, sizeof(float) * csize);
    for (int it = 0; it < iterations; ++it) {
        oracle_center_norms(centers, batch, clusters, dims, norms);
        oracle_assign(x, centers, norms, batch, tokens, dims, clusters, labels, NULL, NULL);
        oracle_update(x, labels, centers, batch, tokens, dims, clusters, sums, counts, means);
        float* tmp = centers; centers = means; means = tmp;
    }
    memcpy(centers_out, centers, sizeof(float) * csize);
    if (indices && offsets) oracle_stable_sort(labels, batch, tokens, clusters, indices, offsets);
    free(centers); free(means); free(sums); free(norms);
}

/* Base-Offset quantizer, encode and decode, per token over all dims:
 *   r = x - C[label]; low = min r; high = max r
 *   scale = (high - low) / (2^bits - 1), or 1 when that is not positive
 *   code = clamp(round_half_even((r - low) / scale), 0, 2^bits - 1)
 *   xhat = C[label] + (low + scale * code)          (fp32; cast to the input dtype by the caller)
 * Each line is one fp32 rounding, in this order (peco/quantization.py:111-118,134-136). */
void oracle_base_offset(const float* x, const int32_t* labels, const float* centroids, int batch,
                        int tokens, int clusters, int dims, int bits, uint8_t* codes, float* low_out,
                        float* scale_out, float* xhat) {
    const float levels = (float)((1 << bits) - 1);
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < (int64_t)batch * tokens; ++row) {
        const int64_t b = row / tokens;
        const float* c = centroids + (b * clusters + labels[row]) * dims;
        const float* xr = x + row * dims;
        float low = INFINITY, high = -INFINITY;
        for (int d = 0; d < dims; ++d) {
            const float r = xr[d] - c[d];
            low = r < low ? r : low;
            high = r > high ? r : high;
        }
        const float span = high - low;
        const float raw = span / levels;
        const float scale = raw > 0.0f ? raw : 1.0f;
        for (int d = 0; d < dims; ++d) {
            const float r = xr[d] - c[d];
            const float shifted = r - low;
            float q = rintf(shifted / scale);
            q = q < 0.0f ? 0.0f : (q > levels ? levels : q);
            const uint8_t code = (uint8_t)q;
            const float step = scale * (float)code;
            const float resid = low + step;
            if (codes) codes[row * dims + d] = code;
            if (xhat) xhat[row * dims + d] = c[d] + resid;
        }
        if (low_out) low_out[row] = low;
        if (scale_out) scale_out[row] = scale;
    }
}

/* Cluster-masked attention in double precision. Query/key rows are grouped by cluster in
 * the order of q_sizes/k_sizes; a size that would run past the sequence is clamped as in
 * peco/kernels/sparse_attention.cu:29,36. Query rows not covered by any cluster, and rows
 * with no selected key, are written as zero. */
void oracle_sparse_attention(const float* q, const float* k, const float* v, const uint8_t* map,
                             const int32_t* q_sizes, const int32_t* k_sizes, int bh, int sq, int sk,
                             int dims, int cq, int ck, float* out) {
    const double scale = 1.0 / sqrt((double)dims);
    memset(out, 0, sizeof(float) * (size_t)bh * sq * dims);
    for (int b = 0; b < bh; ++b) {
        int32_t* kpre = (int32_t*)malloc(sizeof(int32_t) * (size_t)(ck + 1));
        int32_t* qcl = (int32_t*)malloc(sizeof(int32_t) * (size_t)sq);
        int off = 0;
        kpre[0] = 0;
        for (int c = 0; c < ck; ++c) {
            int s = k_sizes[(int64_t)b * ck + c];
            if (s > sk - off) s = sk - off;
            if (s < 0) s = 0;
            off += s;
            kpre[c + 1] = off;
        }
        for (int r = 0; r < sq; ++r) qcl[r] = -1;
        off = 0;
        for (int c = 0; c < cq; ++c) {
            int s = q_sizes[(int64_t)b * cq + c];
            if (s > sq - off) s = sq - off;
            if (s < 0) s = 0;
            for (int r = off; r < off + s; ++r) qcl[r] = c;
            off += s;
        }
#pragma omp parallel
        {
            double* scores = (double*)malloc(sizeof(double) * (size_t)(sk > 0 ? sk : 1));
            double* acc = (double*)malloc(sizeof(double) * (size_t)dims);
#pragma omp for schedule(dynamic, 16)
            for (int r = 0; r < sq; ++r) {
                const int c = qcl[r];
                if (c < 0) continue;
                const uint8_t* sel = map + ((int64_t)b * cq + c) * ck;
                const float* qr = q + ((int64_t)b * sq + r) * dims;
                double m = -INFINITY;
                int n = 0;
                for (int kc = 0; kc < ck; ++kc) {
                    if (!sel[kc]) continue;
                    for (int j = kpre[kc]; j < kpre[kc + 1]; ++j) {
                        const float* kr = k + ((int64_t)b * sk + j) * dims;
                        double s = 0.0;
                        for (int d = 0; d < dims; ++d) s += (double)qr[d] * (double)kr[d];
                        s *= scale;
                        scores[n++] = s;
                        if (s > m) m = s;
                    }
                }
                if (n == 0) continue;
                for (int d = 0; d < dims; ++d) acc[d] = 0.0;
                double l = 0.0;
                n = 0;
                for (int kc = 0; kc < ck; ++kc) {
                    if (!sel[kc]) continue;
                    for (int j = kpre[kc]; j < kpre[kc + 1]; ++j) {
                        const double p = exp(scores[n++] - m);
                        const float* vr = v + ((int64_t)b * sk + j) * dims;
                        l += p;
                        for (int d = 0; d < dims; ++d) acc[d] += p * (double)vr[d];
                    }
                }
                float* o = out + ((int64_t)b * sq + r) * dims;
                for (int d = 0; d < dims; ++d) o[d] = (float)(acc[d] / l);
            }
            free(scores); free(acc);
        }
        free(kpre); free(qcl);
    }
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
