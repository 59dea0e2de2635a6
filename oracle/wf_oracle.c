/*
 * wf_oracle.c -- CPU restatement of Wayfinder's causal top-K retrieval and sparse
 * attention readout.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for libwayfinder_hip.so.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product package never does.
 *
 * What it restates (reference = /root/reference, pure PyTorch):
 *  - wfo_causal_topk_rows: causal_topk(method="fused_causal")
 *      routing_attention/kernels/causal_topk.py:132-171 (_causal_topk_row_blocked: fp32
 *      scores q.k for j <= t, top-k_eff per row) and :37-57 (_finalize_causal_topk: slots
 *      without a causal key get pad index (t + k_eff + s + 1) % T).
 *    The score of (t, j) is defined as the fp32 chain acc = fmaf(q[t,d], k[j,d], acc) over
 *    d = 0..R-1 starting from acc = 0, on inputs converted exactly to fp32 (the reference
 *    casts to fp32 at causal_topk.py:150-151 and lets torch.bmm pick the summation order).
 *    Ties resolve to the lower key index (the north-star rule; the reference's only
 *    explicit tie semantic, the Triton heap at causal_topk.py:305-315 streaming keys in
 *    ascending order, behaves the same). Output is canonical: score descending, then
 *    index ascending; valid keys fill slots 0..n_valid-1 and pads follow, which is the
 *    slot placement torch's GPU topk(sorted=False) gives rows whose tail is -inf.
 *    wfo_causal_topk_rowlist: the same for an explicit list of (b, t) rows.
 *  - wfo_sparse_readout: sparse_meat_attention_reference
 *      routing_attention/kernels/fused_sparse.py:80-94 (gather k/v at indices shared
 *      across heads :64-77, scores = (q . k_sel) * scale, softmax, weighted sum of v_sel),
 *    accumulated in double. Negative indices wrap by +T (torch advanced indexing);
 *    indices outside [-T, T) are clamped to [0, T-1] (the reference raises there).
 *  - wfo_sparse_readout_dropout / wfo_dropout_mask: the reference's non-fused training
 *    readout, routing_attention/models/attention.py:35-55 (attn = dropout(softmax(...))),
 *    with the keep mask defined by a hash of (seed, b, h, t, s) -- the definition of
 *    wf_sparse_readout_fwd_dropout in include/wayfinder_hip.h, restated here; the reference
 *    draws its mask from torch's generator instead, which no implementation reproduces.
 *
 * Build: oracle/Makefile -> oracle/libwf_oracle.so (gcc, OpenMP over rows).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* fp32 score of one (query, key) pair: sequential fused multiply-add chain. */
float wfo_score(const float* q, const float* k, int64_t R)
{
    float acc = 0.0f;
    for (int64_t d = 0; d < R; ++d) acc = fmaf(q[d], k[d], acc);
    return acc;
}

/* Total order used for selection: a is better than b. */
static int better(float sa, int32_t ja, float sb, int32_t jb)
{
    return (sa > sb) || (sa == sb && ja < jb);
}

typedef struct { float s; int32_t j; } cand;

/* min-heap by "better": root is the worst kept candidate */
static void sift_down(cand* h, int64_t n, int64_t i)
{
    for (;;) {
        int64_t l = 2 * i + 1, r = l + 1, w = i;
        if (l < n && better(h[w].s, h[w].j, h[l].s, h[l].j)) w = l;
        if (r < n && better(h[w].s, h[w].j, h[r].s, h[r].j)) w = r;
        if (w == i) return;
        cand t = h[i]; h[i] = h[w]; h[w] = t; i = w;
    }
}

static int cmp_desc(const void* pa, const void* pb)
{
    const cand* a = (const cand*)pa;
    const cand* b = (const cand*)pb;
    if (better(a->s, a->j, b->s, b->j)) return -1;
    if (better(b->s, b->j, a->s, a->j)) return 1;
    return 0;
}

/*
 * Row t of batch b: the k_eff best keys j <= t in canonical order, pads after them.
 * heap: scratch of k_eff candidates. out_idx / out_score: k_eff entries (score may be NULL).
 */
static void topk_row(const float* qa, const float* ka, int64_t T, int64_t R, int64_t k_eff,
                     int64_t b, int64_t t, cand* heap, int32_t* oi, float* os)
{
    const float* q = qa + (b * T + t) * R;
    int64_t n = 0;
    for (int64_t j = 0; j <= t; ++j) {
        const float s = wfo_score(q, ka + (b * T + j) * R, R);
        if (n < k_eff) {
            /* insert and restore heap order upward */
            int64_t i = n++;
            heap[i].s = s; heap[i].j = (int32_t)j;
            while (i > 0) {
                int64_t p = (i - 1) / 2;
                if (better(heap[p].s, heap[p].j, heap[i].s, heap[i].j)) {
                    cand tmp = heap[p]; heap[p] = heap[i]; heap[i] = tmp; i = p;
                } else break;
            }
        } else if (better(s, (int32_t)j, heap[0].s, heap[0].j)) {
            heap[0].s = s; heap[0].j = (int32_t)j;
            sift_down(heap, n, 0);
        }
    }
    qsort(heap, (size_t)n, sizeof(cand), cmp_desc);
    for (int64_t s = 0; s < k_eff; ++s) {
        if (s < n) {
            oi[s] = heap[s].j;
            if (os) os[s] = heap[s].s;
        } else {
            oi[s] = (int32_t)((t + k_eff + s + 1) % T);
            if (os) os[s] = -INFINITY;
        }
    }
}

/*
 * Rows [row0, row1) of batch b. qa, ka: contiguous (B, T, R) fp32.
 * out_idx / out_score: contiguous (row1 - row0, k_eff); out_score may be NULL.
 */
void wfo_causal_topk_rows(const float* qa, const float* ka, int64_t B, int64_t T, int64_t R,
                          int64_t top_k, int64_t b, int64_t row0, int64_t row1,
                          int32_t* out_idx, float* out_score)
{
    (void)B;
    const int64_t k_eff = top_k < T ? top_k : T;
    if (k_eff <= 0) return;
#pragma omp parallel
    {
        cand* heap = (cand*)malloc(sizeof(cand) * (size_t)k_eff);
#pragma omp for schedule(dynamic, 16)
        for (int64_t t = row0; t < row1; ++t)
            topk_row(qa, ka, T, R, k_eff, b, t, heap, out_idx + (t - row0) * k_eff,
                     out_score ? out_score + (t - row0) * k_eff : NULL);
        free(heap);
    }
}

/*
 * Selected rows: rows_bt holds n pairs (b, t). out_idx / out_score: contiguous (n, k_eff);
 * out_score may be NULL.
 */
void wfo_causal_topk_rowlist(const float* qa, const float* ka, int64_t B, int64_t T, int64_t R,
                             int64_t top_k, const int64_t* rows_bt, int64_t n,
                             int32_t* out_idx, float* out_score)
{
    (void)B;
    const int64_t k_eff = top_k < T ? top_k : T;
    if (k_eff <= 0) return;
#pragma omp parallel
    {
        cand* heap = (cand*)malloc(sizeof(cand) * (size_t)k_eff);
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < n; ++i)
            topk_row(qa, ka, T, R, k_eff, rows_bt[2 * i], rows_bt[2 * i + 1], heap,
                     out_idx + i * k_eff, out_score ? out_score + i * k_eff : NULL);
        free(heap);
    }
}

/* All rows of all batches: out_idx / out_score contiguous (B, T, k_eff). */
void wfo_causal_topk(const float* qa, const float* ka, int64_t B, int64_t T, int64_t R,
                     int64_t top_k, int32_t* out_idx, float* out_score)
{
    const int64_t k_eff = top_k < T ? top_k : T;
    for (int64_t b = 0; b < B; ++b)
        wfo_causal_topk_rows(qa, ka, B, T, R, top_k, b, 0, T, out_idx + b * T * k_eff,
                             out_score ? out_score + b * T * k_eff : NULL);
}

/* Dropout keep decision (include/wayfinder_hip.h, wf_sparse_readout_fwd_dropout): the
 * "lowbias32" integer hash (C. Wellons, hash-prospector) chained over the row id
 * r = (b*H + h)*T + t and the seed halves, then over the slot s. */
static uint32_t mix32(uint32_t x)
{
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

static uint32_t drop_threshold(float p)
{
    const double t = floor((double)p * 4294967296.0 + 0.5);
    return t > 4294967295.0 ? 0xffffffffu : (uint32_t)t;
}

static int drop_keep(uint64_t seed, uint64_t row_id, uint32_t slot, uint32_t thresh)
{
    const uint32_t key = mix32(mix32((uint32_t)row_id ^ (uint32_t)seed) ^ (uint32_t)(row_id >> 32) ^
                               (uint32_t)(seed >> 32));
    return mix32(key ^ slot) >= thresh;
}

/* out: contiguous (B, H, T, K) bytes, 1 = kept. */
void wfo_dropout_mask(int64_t B, int64_t H, int64_t T, int64_t K, float p, uint64_t seed,
                      uint8_t* out)
{
    const uint32_t thresh = drop_threshold(p);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < B * H * T; ++r)
        for (int64_t s = 0; s < K; ++s) out[r * K + s] = (uint8_t)drop_keep(seed, (uint64_t)r, (uint32_t)s, thresh);
}

/*
 * One (b, h, t) row of the readout: softmax over the K slots of idx_row of
 * scale * q[b,h,t] . k[b,h,j], weighted sum of v[b,h,j], accumulated in double.
 * q, k, v: contiguous (B, H, T, D) fp32. sc / jj: scratch of K entries.
 * flags bit 0: zero weight for slots s > t of rows t < K - 1 (pad slots of the retrieval).
 * drop_p > 0: after the softmax, weight s is kept if drop_keep(...) and scaled by
 * 1 / (1 - drop_p) (computed in fp32, as the kernels do), else zeroed.
 */
static void readout_row(const float* q, const float* k, const float* v, int64_t H, int64_t T,
                        int64_t D, int64_t b, int64_t h, int64_t t, const int32_t* idx_row,
                        int64_t K, float scale, unsigned flags, float drop_p, uint64_t seed,
                        double* sc, int64_t* jj, double* orow)
{
    const uint32_t thresh = drop_threshold(drop_p);
    const double dscale = (double)(1.0f / (1.0f - drop_p));
    const int64_t bh = b * H + h;
    const float* qr = q + (bh * T + t) * D;
    double m = -INFINITY;
    for (int64_t s = 0; s < K; ++s) {
        int64_t j = idx_row[s];
        if (j < 0) j += T;
        if (j < 0) j = 0;
        if (j > T - 1) j = T - 1;
        jj[s] = j;
        const int masked = (flags & 1u) && t < K - 1 && s > t;
        if (masked) { sc[s] = -INFINITY; continue; }
        const float* kr = k + (bh * T + j) * D;
        double dot = 0.0;
        for (int64_t d = 0; d < D; ++d) dot += (double)qr[d] * (double)kr[d];
        sc[s] = dot * (double)scale;
        if (sc[s] > m) m = sc[s];
    }
    for (int64_t d = 0; d < D; ++d) orow[d] = 0.0;
    double l = 0.0;
    for (int64_t s = 0; s < K; ++s) {
        if (sc[s] == -INFINITY) continue;
        const double p = exp(sc[s] - m);
        l += p;
        double w = p;
        if (drop_p > 0.0f)
            w = drop_keep(seed, (uint64_t)(bh * T + t), (uint32_t)s, thresh) ? p * dscale : 0.0;
        const float* vr = v + (bh * T + jj[s]) * D;
        for (int64_t d = 0; d < D; ++d) orow[d] += w * (double)vr[d];
    }
    for (int64_t d = 0; d < D; ++d) orow[d] = l > 0.0 ? orow[d] / l : 0.0;
}

/*
 * q, k, v: contiguous (B, H, T, D) fp32; idx: contiguous (B, T, K) int32;
 * out: contiguous (B, H, T, D) double (readout_row for every row).
 */
void wfo_sparse_readout_dropout(const float* q, const float* k, const float* v,
                                int64_t B, int64_t H, int64_t T, int64_t D,
                                const int32_t* idx, int64_t K, float scale, unsigned flags,
                                float drop_p, uint64_t seed, double* out)
{
#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
        int64_t* jj = (int64_t*)malloc(sizeof(int64_t) * (size_t)(K > 0 ? K : 1));
#pragma omp for collapse(2) schedule(static)
        for (int64_t bh = 0; bh < B * H; ++bh) {
            for (int64_t t = 0; t < T; ++t) {
                const int64_t b = bh / H, h = bh % H;
                readout_row(q, k, v, H, T, D, b, h, t, idx + (b * T + t) * K, K, scale, flags,
                            drop_p, seed, sc, jj, out + (bh * T + t) * D);
            }
        }
        free(sc);
        free(jj);
    }
}

/* wfo_sparse_readout_dropout without dropout. */
void wfo_sparse_readout(const float* q, const float* k, const float* v,
                        int64_t B, int64_t H, int64_t T, int64_t D,
                        const int32_t* idx, int64_t K, float scale, unsigned flags,
                        double* out)
{
    wfo_sparse_readout_dropout(q, k, v, B, H, T, D, idx, K, scale, flags, 0.0f, 0, out);
}

/*
 * Selected rows only (cheap checks at full T): rows_bt holds n pairs (b, t); idx is
 * contiguous (n, K) (the index row of each pair); out is contiguous (n, H, D) double.
 */
void wfo_sparse_readout_rows(const float* q, const float* k, const float* v,
                             int64_t B, int64_t H, int64_t T, int64_t D,
                             const int64_t* rows_bt, int64_t n, const int32_t* idx, int64_t K,
                             float scale, unsigned flags, double* out)
{
    (void)B;
#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
        int64_t* jj = (int64_t*)malloc(sizeof(int64_t) * (size_t)(K > 0 ? K : 1));
#pragma omp for collapse(2) schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            for (int64_t h = 0; h < H; ++h)
                readout_row(q, k, v, H, T, D, rows_bt[2 * i], h, rows_bt[2 * i + 1], idx + i * K,
                            K, scale, flags, 0.0f, 0, sc, jj, out + (i * H + h) * D);
        }
        free(sc);
        free(jj);
    }
}
