/*
 * wayfinder_hip.h -- C ABI of libwayfinder_hip.so, the MI355X (gfx950) implementation of
 * Wayfinder's causal top-K address retrieval plus sparse ("meat") attention forward.
 *
 * Every entry point replaces one function of the reference's Python kernel layer
 * (routing_attention/kernels/, pure PyTorch there); the reference file:line each one
 * stands in for is given beside it. The reference has no FFI of its own: the binding a
 * maintainer would add on the reference side is a ctypes stub.
 *
 * Conventions
 *  - All tensor arguments are device pointers (hipMalloc'd or from the PyTorch caching
 *    allocator). Shapes and strides are in ELEMENTS, int64. The library never allocates,
 *    frees or keeps a pointer after the call returns; the caller owns every buffer,
 *    including the optional workspace.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream). Work is enqueued
 *    asynchronously; no entry point synchronises the host.
 *  - Return value: WF_OK (0) or a wf_status code. The message of the last failure on the
 *    calling thread is available from wf_last_error(). Argument validation happens before
 *    any HIP call, so contract errors are reported even on a machine without a GPU.
 *  - Indices are int32. Index sets are emitted in canonical order: score descending, ties
 *    to the lower key index, pad slots last. The reference returns an unspecified order
 *    (torch.topk(sorted=False)); compare as sets.
 */
#ifndef WAYFINDER_HIP_H
#define WAYFINDER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WF_ABI_VERSION 5

typedef enum wf_status {
    WF_OK = 0,
    WF_ERR_INVALID_ARGUMENT = 1, /* shape / rank / stride / pointer contract violated  */
    WF_ERR_UNSUPPORTED = 2,      /* valid request outside what the kernels implement   */
    WF_ERR_WORKSPACE = 3,        /* workspace missing or smaller than required         */
    WF_ERR_HIP = 4               /* a HIP runtime call or kernel launch failed         */
} wf_status;

typedef enum wf_dtype {
    WF_DTYPE_F32 = 0,
    WF_DTYPE_F16 = 1,
    WF_DTYPE_BF16 = 2
} wf_dtype;

/* Readout flags (wf_sparse_readout_fwd / wf_fused_args.flags). */
#define WF_FLAG_MASK_PADS 0x1u /* slots s > t of rows t < k_eff-1 (the pad slots written
                                  by the retrieval) get zero weight. Off = reference
                                  behaviour: pads are attended (causal_topk.py:37-57). */

/* Fused-forward pass selection (wf_fused_args.flags). Without either, the library picks. */
#define WF_FLAG_SPLIT_PASS 0x2u  /* retrieval kernel, then readout kernel                      */
#define WF_FLAG_SINGLE_PASS 0x4u /* one kernel: each workgroup retrieves 16 query rows and reads
                                    them out for every head (WF_ERR_UNSUPPORTED unless bf16,
                                    R = 32, 64 < k_eff <= 256, D in {64, 128}, H * D in
                                    {512, 1024}, 16-byte aligned rows, contiguous head dim)     */

/* Library ABI version (WF_ABI_VERSION of the build). No reference counterpart. */
int wf_abi_version(void);

/* Message of the last failed call on this thread ("" if none). No reference counterpart. */
const char* wf_last_error(void);

/* Number of bytes of device workspace wf_causal_topk_fwd needs for this shape
 * (the per-chunk key magnitude bounds of the screening stage). */
size_t wf_causal_topk_workspace_bytes(int64_t B, int64_t T, int64_t R, int64_t top_k);

/*
 * Causal top-K retrieval.
 * Replaces: causal_topk (routing_attention/kernels/causal_topk.py:470-521) with
 *           method auto/fused_causal -> _causal_topk_row_blocked (:132-171) and
 *           _finalize_causal_topk (:37-57).
 * query, key : (B, T, R) of `dtype`, element strides q_strides[3], k_strides[3].
 * out_idx    : (B, T, k_eff) int32, contiguous, k_eff = min(top_k, T).
 *              Row t holds the k_eff keys j <= t with the largest fp32 scores
 *              s(t, j) = fma-chain over d of query[t,d]*key[j,d] (d ascending, fp32),
 *              ties resolved to the lower j. Rows with t+1 < k_eff hold their t+1 causal
 *              keys in slots 0..t and pad index (t + k_eff + s + 1) % T in slot s > t.
 * out_scores : optional (B, T, k_eff) float32 (NULL to skip): the fp32 score of every
 *              slot, -inf in pad slots.
 * workspace  : device buffer of at least wf_causal_topk_workspace_bytes(...) bytes.
 * Limits: 1 <= R <= 256, 1 <= top_k (k_eff <= 512), T < 2^31.
 */
int wf_causal_topk_fwd(const void* query, const void* key, int dtype,
                       int64_t B, int64_t T, int64_t R,
                       const int64_t* q_strides, const int64_t* k_strides,
                       int64_t top_k, int32_t* out_idx, float* out_scores,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Sparse attention readout over pre-selected indices, shared across heads.
 * Replaces: sparse_meat_attention (routing_attention/kernels/fused_sparse.py:275-324),
 *           i.e. _sparse_meat_batched (:97-128) / sparse_meat_attention_reference (:80-94).
 * q, k, v  : (B, H, T, D) of `dtype`, element strides *_strides[4] (any layout; the
 *            (B,T,H,D) memory of a .view(B,T,H,D).transpose(1,2) is the fast case).
 * indices  : (B, T, K) int32, strides idx_strides[3]. Negative entries wrap (+T) as in
 *            torch advanced indexing; entries outside [-T, T) are clamped to [0, T-1].
 * out      : (B, H, T, D) of `dtype`, strides out_strides[4]:
 *            out[b,h,t] = sum_s softmax_s(scale * q[b,h,t].k[b,h,idx[b,t,s]]) v[b,h,idx[b,t,s]]
 *            computed in fp32, rounded once to `dtype`.
 * flags    : WF_FLAG_MASK_PADS or 0.
 * Limits: 1 <= D <= 256, 1 <= K <= 1024.
 */
int wf_sparse_readout_fwd(const void* q, const void* k, const void* v, int dtype,
                          int64_t B, int64_t H, int64_t T, int64_t D,
                          const int64_t* q_strides, const int64_t* k_strides,
                          const int64_t* v_strides,
                          const int32_t* indices, const int64_t* idx_strides, int64_t K,
                          float scale, unsigned flags,
                          void* out, const int64_t* out_strides, void* stream);

/*
 * wf_sparse_readout_fwd that also writes the softmax normaliser the backward needs.
 * Replaces: the forward half of the reference's differentiable readout (attention.py:35-55,
 *           whose gather formulation autograd differentiates).
 * lse2 : (B, H, T) float32, contiguous: log2 of the softmax denominator of every row in
 *        the base-2 domain, lse2 = log2(sum_s 2^(log2(e) * scale * q.k_s)) = lse * log2(e).
 * Other arguments and limits as wf_sparse_readout_fwd.
 */
int wf_sparse_readout_fwd_lse(const void* q, const void* k, const void* v, int dtype,
                              int64_t B, int64_t H, int64_t T, int64_t D,
                              const int64_t* q_strides, const int64_t* k_strides,
                              const int64_t* v_strides,
                              const int32_t* indices, const int64_t* idx_strides, int64_t K,
                              float scale, unsigned flags,
                              void* out, const int64_t* out_strides, float* lse2, void* stream);

/* Arguments of the readout backward. */
typedef struct wf_readout_bwd_args {
    const void* q;              /* (B, H, T, D) forward inputs, strides *_strides  */
    const void* k;
    const void* v;
    const void* dout;           /* (B, H, T, D) gradient of the forward output      */
    const int32_t* indices;     /* (B, T, K) int32, idx_strides[2] == 1             */
    const float* lse2;          /* (B, H, T) from wf_sparse_readout_fwd_lse         */
    void* dq;                   /* (B, H, T, D) outputs, every element written      */
    void* dk;
    void* dv;
    void* workspace;            /* >= wf_sparse_readout_bwd_workspace_bytes(...)    */
    size_t workspace_bytes;
    int64_t q_strides[4];
    int64_t k_strides[4];
    int64_t v_strides[4];
    int64_t dout_strides[4];
    int64_t dq_strides[4];
    int64_t dk_strides[4];
    int64_t dv_strides[4];
    int64_t idx_strides[3];
    int64_t B, H, T, D, K;
    int dtype;                  /* wf_dtype of every (B, H, T, D) tensor */
    float scale;
    unsigned flags;             /* WF_FLAG_MASK_PADS as in the forward   */
} wf_readout_bwd_args;

/* Device workspace of wf_sparse_readout_bwd for this shape (0 and wf_last_error() set if it
 * cannot be sized, e.g. no device). */
size_t wf_sparse_readout_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t K);

/*
 * Backward of the sparse readout with the indices held fixed.
 * Replaces: the autograd backward of the reference's differentiable readout
 *           (attention.py:35-55, _gather_kv_heads :58-69): dq, and dk/dv accumulated over
 *           every (row, slot) that selected a key (duplicates counted per slot).
 * With p the forward's softmax weights, dp_s = dout . v_s, delta = sum_s p_s dp_s:
 *   dq_t = scale sum_s p_s (dp_s - delta) k_s,  dk_j = scale sum p_s (dp_s - delta_t) q_t,
 *   dv_j = sum p_s dout_t   (sums over the (t, s) with index j for dk, dv).
 * fp32 accumulation, deterministic (no floating-point atomics), one rounding per element.
 * Layout: every (B, H, T, D) tensor with contiguous head dim, 16-byte aligned rows and a
 * per-(b, h) span below 4 GiB (the (B, T, H, D) memory of the module qualifies);
 * otherwise WF_ERR_UNSUPPORTED. Limits: D a multiple of 8 up to 256, 1 <= K <= 1024,
 * B*T*K < 2^32.
 */
int wf_sparse_readout_bwd(const wf_readout_bwd_args* args, void* stream);

/*
 * Training forward of the readout with dropout on the attention weights.
 * Replaces: the reference's non-fused training readout (routing_attention/models/attention.py:
 *           35-55): attn = dropout(softmax(scale q.k_s)); out = sum_s attn_s v_s.
 * Weight s of row t of head h in batch b is kept with probability 1 - dropout_p and scaled
 * by 1 / (1 - dropout_p). The keep decision is a counter-based hash of (seed, b, h, t, s):
 *   key  = mix(mix(lo32(r) ^ lo32(seed)) ^ hi32(r) ^ hi32(seed)),  r = (b*H + h)*T + t,
 *   keep = mix(key ^ s) >= round(dropout_p * 2^32),
 * with mix the "lowbias32" integer hash (x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15;
 * x *= 0x846ca68b; x ^= x >> 16). The same seed gives the same mask, so the backward (below)
 * recomputes it instead of storing it. lse2 (required) is the log-sum-exp of the undropped
 * weights, as wf_sparse_readout_fwd_lse writes it. dropout_p in [0, 1): 0 is the plain
 * training forward. Other arguments and limits as wf_sparse_readout_fwd_lse.
 */
int wf_sparse_readout_fwd_dropout(const void* q, const void* k, const void* v, int dtype,
                                  int64_t B, int64_t H, int64_t T, int64_t D,
                                  const int64_t* q_strides, const int64_t* k_strides,
                                  const int64_t* v_strides,
                                  const int32_t* indices, const int64_t* idx_strides, int64_t K,
                                  float scale, unsigned flags, float dropout_p, uint64_t seed,
                                  void* out, const int64_t* out_strides, float* lse2, void* stream);

/*
 * Backward of wf_sparse_readout_fwd_dropout (same dropout_p and seed, hence the same mask m):
 * as wf_sparse_readout_bwd with dp_s = m_s / (1 - dropout_p) * (dout . v_s) and
 * dv_j = sum p_s m_s / (1 - dropout_p) dout_t. Arguments and limits as wf_sparse_readout_bwd.
 */
int wf_sparse_readout_bwd_dropout(const wf_readout_bwd_args* args, float dropout_p, uint64_t seed,
                                  void* stream);

/*
 * Learned-address projection and L2 normalisation, both address streams in one pass.
 * Replaces: LearnedAddressModule.forward_query_key
 *           (routing_attention/models/learned_address.py:39-46):
 *           q = normalize(x Wq^T + bq), k = normalize(x Wk^T + bk) (normalize = x / max(|x|, 1e-12)).
 * x           : (B, T, d_model) of `dtype`, strides x_strides[3] (x_strides[2] == 1, 16-byte
 *               aligned rows).
 * wq, wk      : (R, d_model) nn.Linear weights of `dtype`, row stride w_stride (16-byte aligned
 *               rows, unit column stride); bq, bk: (R) biases or NULL. wk == NULL: symmetric,
 *               only out_q is written.
 * out_q/out_k : (B, T, R) of `dtype`, strides oq_strides / ok_strides.
 * normalize   : 0 = projections only.
 * Rounding follows the PyTorch ops replaced: the projection is rounded to `dtype` (bias
 * added in fp32), the norm of the rounded values accumulated in fp32 and rounded, the
 * quotient computed in fp32 and rounded once. Limits: 1 <= R <= 32, d_model % 8 == 0.
 */
int wf_address_project_fwd(const void* x, int dtype, int64_t B, int64_t T, int64_t d_model,
                           const int64_t* x_strides, const void* wq, const void* bq,
                           const void* wk, const void* bk, int64_t w_stride, int64_t R,
                           int normalize, void* out_q, const int64_t* oq_strides,
                           void* out_k, const int64_t* ok_strides, void* stream);

/*
 * Residual add + LayerNorm over the last dim, one pass.
 * Replaces: in TransformerBlock.forward (routing_attention/models/transformer.py:50-73) and
 *           the final norm (transformer.py:332), the pair `x = x + delta` followed by
 *           nn.LayerNorm(x) (F.layer_norm, biased variance).
 * x, delta    : (rows, n) of `dtype` at row strides x_stride / delta_stride (unit column
 *               stride, 16-byte aligned rows); delta == NULL: LayerNorm of x alone.
 * weight, bias: (n) of `dtype`, 16-byte aligned, or NULL (no affine scale / shift).
 * sum_out     : x + delta, rounded to `dtype`, at sum_stride, or NULL (not written; also not
 *               written when delta == NULL).
 * y           : LayerNorm(x + delta) at y_stride: (s - mean) / sqrt(var + eps) * weight +
 *               bias over each row of s = x + delta, computed in fp32 and rounded once.
 * Limits: n % 8 == 0, n <= 1024. sum_out and y may not overlap x or delta.
 */
int wf_residual_layernorm_fwd(const void* x, const void* delta, int dtype, int64_t rows, int64_t n,
                              int64_t x_stride, int64_t delta_stride, const void* weight,
                              const void* bias, float eps, void* sum_out, int64_t sum_stride,
                              void* y, int64_t y_stride, void* stream);

/* Arguments of the fused forward, one struct so the entry point stays stable. */
typedef struct wf_fused_args {
    const void* q_search;       /* (B, T, R) addresses, strides qs_strides  */
    const void* k_search;       /* (B, T, R) addresses, strides ks_strides  */
    const void* q;              /* (B, H, T, D), strides q_strides          */
    const void* k;
    const void* v;
    void* out;                  /* (B, H, T, D), strides out_strides        */
    int32_t* out_idx;           /* (B, T, k_eff) int32 contiguous           */
    float* out_scores;          /* optional (B, T, k_eff) fp32, or NULL     */
    void* workspace;            /* >= wf_fused_workspace_bytes(...)         */
    size_t workspace_bytes;
    int64_t qs_strides[3];
    int64_t ks_strides[3];
    int64_t q_strides[4];
    int64_t k_strides[4];
    int64_t v_strides[4];
    int64_t out_strides[4];
    int64_t B, H, T, D, R, top_k;
    int search_dtype;           /* wf_dtype of q_search/k_search */
    int dtype;                  /* wf_dtype of q/k/v/out         */
    float scale;
    unsigned flags;             /* WF_FLAG_* */
} wf_fused_args;

size_t wf_fused_workspace_bytes(int64_t B, int64_t T, int64_t R, int64_t top_k);

/*
 * Fused causal top-K retrieval + sparse attention forward.
 * Replaces: fused_sparse_attention (routing_attention/kernels/fused_sparse.py:327-356):
 *           causal_topk(q_search, k_search, top_k) then sparse_meat_attention(q, k, v,
 *           indices, scale); writes both the output and the indices.
 */
int wf_fused_topk_sparse_fwd(const wf_fused_args* args, void* stream);

/*
 * wf_fused_topk_sparse_fwd for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. Same arguments, results and errors as wf_fused_topk_sparse_fwd except that
 * args->workspace / workspace_bytes are ignored: the retrieval's scratch (B * ceil(T / 256)
 * floats) comes from a 1 MiB array the library keeps on each device until the process ends,
 * so shapes with B * ceil(T / 256) > 262144 are rejected (WF_ERR_UNSUPPORTED). Calls no
 * allocating routine. Calls that overlap on one device share that array and race: issue
 * them on one stream, or serialise them.
 */
size_t wf_fused_noalloc_scratch_limit(void);
int wf_fused_topk_sparse_fwd_noalloc(const wf_fused_args* args, void* stream);

/*
 * Measurement aid, no reference counterpart: the readout's gather path with no arithmetic.
 * Issues exactly the loads of wf_sparse_readout_fwd's fast kernel (same grid, workgroup
 * order, 16-byte index loads and K/V row gathers, two tasks in flight per wave) and folds
 * the loaded words into one XOR per lane written to `sink`, so its time is the speed of
 * light of the readout's memory pattern. k, v: (B, H, T, D) bf16/f16 in the readout's fast
 * layout; indices (B, T, K) int32 with contiguous, 16-byte aligned rows, K % 4 == 0 (entries
 * are clamped to [0, T-1]); sink: >= wf_probe_gather_sink_bytes(B, H, T) bytes.
 */
size_t wf_probe_gather_sink_bytes(int64_t B, int64_t H, int64_t T);
int wf_probe_gather(const void* k, const void* v, int dtype, int64_t B, int64_t H, int64_t T,
                    int64_t D, const int64_t* k_strides, const int64_t* v_strides,
                    const int32_t* indices, const int64_t* idx_strides, int64_t K,
                    uint32_t* sink, size_t sink_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WAYFINDER_HIP_H */
