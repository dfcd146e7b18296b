/*
 * nq_attn.h -- C ABI of the gfx950 (MI355X) GQA attention library
 * (libnqattn.so), a drop-in for nano-qwen's attention hot path.
 *
 * Conventions shared by every entry point
 *   - All tensor pointers are HIP device pointers; the caller owns every
 *     buffer (including the decode workspace).  Nothing here allocates,
 *     frees or synchronises.  Launches go on `stream` (a hipStream_t; NULL =
 *     the default stream).
 *   - A "row" is head_dim contiguous elements.  4-D tensors are described by
 *     their base pointer plus three element strides for the (batch, head,
 *     sequence) axes; the head_dim axis must be contiguous.  Base pointers must
 *     be 16-byte aligned and strides multiples of 16 bytes.  So must the fp32
 *     cos/sin tables given to nq_attn_prefill_fwd (rows go to LDS by DMA).
 *   - dtype codes: NQ_DTYPE_BF16 (bfloat16 stored as 16-bit words) or
 *     NQ_DTYPE_F32.  bf16 data: matrix products on bf16 MFMA with fp32
 *     accumulation.  fp32 data in nq_attn_prefill_fwd: products on fp32 MFMA
 *     (the reference's SDPA keeps the input dtype).  Norm, RoPE and softmax
 *     arithmetic is fp32 everywhere.
 *   - head_dim must be 32, 64 or 128 (the reference's configs use 32 and 128).
 *     kernels/flash_attn.py:106 also allows 16 and 256: nq_attn_prefill_fwd
 *     and nq_attn_bwd take 256 for plain bf16 attention (no QK-Norm/RoPE
 *     fusion, key lengths or bias); 16 is refused here with
 *     NQ_ERR_UNSUPPORTED (the Python wrapper pads it to 32).  num_heads % num_kv_heads == 0 and query
 *     head h reads kv head h / (num_heads / num_kv_heads).
 *   - cos/sin tables are fp32 (max_pos, head_dim/2) row-major, as built by the
 *     reference's RotaryEmbedding (plain RoPE or YaRN).  A row rotated at a
 *     position outside [0, max_pos) comes out NaN (the reference's table
 *     lookup, model/rope.py:123-129, fails there; positions held on the
 *     device cannot be reported from a kernel, so callers that know them on
 *     the host check them there).
 *   - Return value: NQ_OK (0) on success, a positive NQ_ERR_* code for an
 *     argument error, or a negative value -(hipError_t) for a launch error.
 *     nq_last_error() returns a thread-local message for the last failure.
 */
#ifndef NQ_ATTN_H_
#define NQ_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NQ_OK 0
#define NQ_ERR_INVALID 1
#define NQ_ERR_UNSUPPORTED 2
#define NQ_ERR_WORKSPACE 3

#define NQ_DTYPE_BF16 0
#define NQ_DTYPE_F32 1

/* Library version, e.g. 100 for 0.1.0. */
int nq_version(void);

/* Thread-local text of the last error ("" when the last call succeeded). */
const char* nq_last_error(void);

/*
 * QK-Norm + RoPE over rows of Q and K, plus an optional row copy of V.
 *
 * Replaces model/norm.py:17-22 (RMSNorm as QK-Norm, applied at
 * model/attention.py:95-97), model/rope.py:133-161 (apply_rotary_pos_emb) and
 * kernels/rope.py:99-108 (apply_rope: in-place when q_out == q, k_out == k),
 * and the concatenation in KVCache.update (model/attention.py:31-38): K and V
 * rows land at destination row kv_row_base[b] + s of a preallocated
 * (B, Hkv, T_cap, D) cache.
 *
 * q, k, v: source rows (any of them NULL to skip that job), with strides
 *   {batch, head, seq} in elements; Q has Hq heads, K and V have Hkv heads.
 * q_out/k_out/v_out: destinations with their strides; Q rows land at row s.
 * q_weight/k_weight: fp32 RMSNorm weights (D), NULL = no norm (qk_norm=False).
 * cos_tab/sin_tab: fp32 RoPE tables, NULL = no rotation (norm or copy only).
 * eps: RMSNorm epsilon (config.rms_norm_eps).
 * pos: int32 (B, S) positions, or NULL to use pos_base[b] + s, or with
 *   pos_base NULL too, pos0 + s (pos0 = 0 is the reference's
 *   position_ids=None, model/rope.py:123-126).
 * kv_row_base: int32 (B) cache row offsets for K/V, or NULL to use kv_row0.
 */
int nq_qk_norm_rope(const void* q, const int64_t* q_strides, void* q_out,
                    const int64_t* q_out_strides, const void* k, const int64_t* k_strides,
                    void* k_out, const int64_t* k_out_strides, const void* v,
                    const int64_t* v_strides, void* v_out, const int64_t* v_out_strides,
                    int B, int S, int Hq, int Hkv, int D, int dtype_in, int dtype_out,
                    const float* q_weight, const float* k_weight, float eps,
                    const float* cos_tab, const float* sin_tab, int max_pos,
                    const int32_t* pos, const int32_t* pos_base, int pos0,
                    const int32_t* kv_row_base, int kv_row0, void* stream);

/*
 * RMSNorm over rows of `width` elements (a multiple of 8): the forward of
 * model/norm.py:11-22 (RMSNorm, used as QK-Norm at model/attention.py:95-97
 * and as the layer norms of model/transformer.py), with its cast order and
 * dtype promotion: y = (x * rsqrt(mean(x^2) + eps)) rounded to x's dtype, times
 * weight, stored in the promoted dtype of x and weight (bf16 only when both
 * are bf16; dtype_y must be that dtype).  x and y are `rows` rows with the
 * given row strides (elements); weight has `width` contiguous elements.
 */
int nq_rmsnorm(const void* x, int64_t x_row_stride, const void* weight, void* y,
               int64_t y_row_stride, int64_t rows, int width, int dtype_x, int dtype_w,
               int dtype_y, float eps, void* stream);

/*
 * Causal / full GQA prefill attention (FlashAttention-2 style forward).
 *
 * Replaces kernels/flash_attn.py:130-143 (flash_attention) and the
 * post-projection part of Attention.forward, model/attention.py:95-115:
 * QK-Norm and RoPE on Q are fused into the Q load (when q_weight or cos_tab is
 * given), the K/V operands are used as stored (for the reference path, K is
 * already normalised and rotated by nq_qk_norm_rope, V raw), the GQA
 * expansion of attention.py:106-108 is implicit, and SDPA is replaced.
 *
 * q: (B, Hq, S, D) with strides q_strides; k, v: (B, Hkv, T, D); o: output
 *   (B, Hq, S, D) with strides o_strides (pass the strides of a (B, S, Hq, D)
 *   buffer to get o_proj's input layout directly).  q, k, v and o all use
 *   `dtype`; NQ_DTYPE_F32 runs every product in fp32 (v_mfma_f32_32x32x2_f32).
 * lse: optional fp32 (B, Hq, S) natural-log sum-exp of the scaled scores.
 * key_lens: optional int32 (B): sequence b attends only keys
 *   [0, key_lens[b]) -- the key-padding mask SDPA applies for a right-padded
 *   batch (model/attention.py:110-114 with a (B, 1, 1, T) keep-mask, the
 *   reward model's padding, training/reward_model.py:45).  0 gives zero rows,
 *   a value outside [0, T] NaN rows (lse -inf).  NULL = all T keys.
 * q_weight: RMSNorm weight for Q (NULL = none); cos_tab/sin_tab: RoPE table
 *   for Q (NULL = none); q_pos / q_pos_base / q_pos0: Q positions as in
 *   nq_qk_norm_rope.
 * causal: query i sees key j iff j <= i + (T - S) (top-left == bottom-right
 *   when S == T, which is SDPA's is_causal in the reference).
 * sm_scale <= 0 selects 1/sqrt(D), SDPA's default (attention.py:110).
 * Requires 256 % (Hq / Hkv) == 0 (fp32: 128 % (Hq / Hkv) == 0) and S <= T
 * when causal.
 */
int nq_attn_prefill_fwd(const void* q, const int64_t* q_strides, const void* k,
                        const int64_t* k_strides, const void* v, const int64_t* v_strides,
                        void* o, const int64_t* o_strides, float* lse, const int32_t* key_lens,
                        int B, int Hq, int Hkv,
                        int S, int T, int D, int dtype, const float* q_weight, float eps,
                        const float* cos_tab, const float* sin_tab, int max_pos,
                        const int32_t* q_pos, const int32_t* q_pos_base, int q_pos0,
                        int causal, float sm_scale, void* stream);

/*
 * nq_attn_prefill_fwd with a general attention mask as an additive bias.
 *
 * Replaces SDPA's attn_mask at model/attention.py:110-113 (passed by callers
 * such as training/reward_model.py:45): a bool keep-mask (True = attend) is
 * given as 0 / -inf, a float mask as its values, both in `dtype`.
 * bias[b, h, i, j] lies at bias + b * bias_strides[0] + h * bias_strides[1] +
 * i * bias_strides[2] + j (element strides; 0 broadcasts an axis); every
 * row's keys are contiguous and readable up to T rounded up to a multiple of
 * 8; the base is 16-byte aligned and the strides are non-negative multiples
 * of 8.  The bias adds to scale * q.k before the softmax; key_lens and causal
 * still apply.  A row whose keys are all masked gets zeros and LSE -inf (as
 * SDPA gives).  Requires 128 % (Hq / Hkv) == 0.  Other arguments as
 * nq_attn_prefill_fwd.
 */
int nq_attn_prefill_bias_fwd(const void* q, const int64_t* q_strides, const void* k,
                             const int64_t* k_strides, const void* v, const int64_t* v_strides,
                             void* o, const int64_t* o_strides, float* lse, const int32_t* key_lens,
                             const void* bias, const int64_t* bias_strides, int B, int Hq, int Hkv,
                             int S, int T, int D, int dtype, const float* q_weight, float eps,
                             const float* cos_tab, const float* sin_tab, int max_pos,
                             const int32_t* q_pos, const int32_t* q_pos_base, int q_pos0, int causal,
                             float sm_scale, void* stream);

/*
 * nq_attn_prefill_fwd over K/V held in paged pools: a chunk of S new queries
 * attends the T keys of its sequence (the T - S already cached plus the S just
 * appended), read through the block table, so a chunked prefill into a paged
 * cache never gathers the pages into a dense copy.
 *
 * Replaces the concatenation of KVCache.update (model/attention.py:31-38)
 * followed by SDPA over the whole cache (attention.py:105-115) for a
 * continuation of the prompt; the reference has no paged cache (the pool
 * format is the one nq_attn_decode_paged_fwd reads).
 *
 * k_pool/v_pool: (num_pages, Hkv, page_size, D) with strides {page, head,
 *   row}; key t of sequence b is row t % page_size of page
 *   block_table[b * bt_stride + t / page_size].  page_size % 32 == 0 and
 *   bt_stride >= ceil(T / page_size).  Every sequence holds T keys.
 * The other arguments are those of nq_attn_prefill_fwd (no key_lens);
 * causal keeps key j for query i iff j <= i + T - S.
 */
int nq_attn_prefill_paged_fwd(const void* q, const int64_t* q_strides, const void* k_pool,
                              const int64_t* k_pool_strides, const void* v_pool,
                              const int64_t* v_pool_strides, const int32_t* block_table,
                              int64_t bt_stride, int page_size, void* o, const int64_t* o_strides,
                              float* lse, int B, int Hq, int Hkv, int S, int T, int D, int dtype,
                              const float* q_weight, float eps, const float* cos_tab,
                              const float* sin_tab, int max_pos, const int32_t* q_pos,
                              const int32_t* q_pos_base, int q_pos0, int causal, float sm_scale,
                              void* stream);

/*
 * Bytes of fp32 workspace nq_attn_decode_fwd needs for these sizes (no
 * counterpart in the reference, whose decode allocates inside torch).
 * max_len bounds every lens[b].  chunk = 0 spreads the cache evenly over a
 * persistent grid sized to the device; chunk > 0 gives every wave chunk keys
 * (rounded up to a multiple of 32) of the concatenated rows instead.
 */
int64_t nq_attn_decode_workspace_bytes(int B, int Hq, int Hkv, int D, int max_len, int chunk);

/*
 * Single-token decode attention against a ragged KV cache.
 *
 * Replaces model/attention.py:95-115 at S == 1 with a KVCache: the new
 * token's Q is QK-Normed and rotated in the kernel (q_weight / cos_tab may be
 * NULL), then attends keys [0, lens[b]) of the cache with no causal mask
 * (attention.py:113 sets is_causal=False whenever a cache is present).
 *
 * q: (B, Hq, D) with strides {batch, head}; k_cache/v_cache: (B, Hkv, T_cap, D)
 *   with strides {batch, head, seq}, holding post-norm post-RoPE K and raw V.
 * lens: int32 (B), 0 <= lens[b] <= max_len <= T_cap; NULL = every row has
 *   max_len keys.  A row with no keys gets zeros; a row whose lens[b] lies
 *   outside [0, max_len] attends nothing and gets NaN.
 * q_pos: int32 (B) RoPE positions of the query token; NULL = q_pos0 for
 *   every row, or lens[b] - 1 when q_pos0 < 0.
 * o: output (B, Hq, D) with strides {batch, head}.
 * workspace: device buffer of at least
 *   nq_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, chunk) bytes for
 *   bf16 caches; fp32 caches keep no partials and ignore it (NULL allowed).
 * Requires Hq / Hkv <= 16 or a multiple of 16.
 */
int nq_attn_decode_fwd(const void* q, const int64_t* q_strides, const void* k_cache,
                       const int64_t* k_strides, const void* v_cache, const int64_t* v_strides,
                       const int32_t* lens, void* o, const int64_t* o_strides, void* workspace,
                       int64_t workspace_bytes, int B, int Hq, int Hkv, int D, int max_len,
                       int chunk, int dtype, const float* q_weight, float eps,
                       const float* cos_tab, const float* sin_tab, int max_pos,
                       const int32_t* q_pos, int q_pos0, float sm_scale, void* stream);

/*
 * Paged KV caches.  A pool of pages (pages, Hkv, page_size, D), described by
 * strides {page, head, row}; row t of sequence b is row t % page_size of page
 * block_table[b * bt_stride + t / page_size] (int32 page ids).  A dense
 * (B, Hkv, T_cap, D) cache is the pool of B pages of T_cap rows with the
 * block table {0, 1, ..., B-1} and bt_stride 1.
 *
 * The reference has no paged cache: these replace the dense per-layer
 * KVCache (model/attention.py:24-46) for batched serving, with the same
 * contents (post-norm post-RoPE K, raw V).
 */

/*
 * Single-token decode against a paged cache, with the new token's K/V append
 * fused in (model/attention.py:95-115 at S == 1, plus KVCache.update,
 * attention.py:31-38, in one launch).
 *
 * Without k_new (NULL): as nq_attn_decode_fwd, over keys [0, lens[b]) read
 *   through the block table; lens is required.
 * With k_new/v_new ((B, Hkv, D), strides {batch, head}, the projection
 *   output before QK-Norm / RoPE): the new key is normed with k_weight (NULL =
 *   no norm) and rotated at the query's position, written with v_new to row
 *   lens[b] of the cache (its page must be mapped), and attended together with
 *   keys [0, lens[b]).  The query position is q_pos[b], else q_pos0, else
 *   lens[b].  lens_out (may be NULL; must not alias lens) receives lens + 1.
 *   A sequence whose lens[b] + 1 exceeds max_len (or lens[b] < 0) appends
 *   nothing, keeps lens_out[b] = lens[b] and gets NaN output.
 *   Calls that overlap on one sequence race; a single call is race-free.
 * max_len bounds the keys attended per sequence (the appended one included)
 *   and sizes the workspace (nq_attn_decode_workspace_bytes); bt_stride must
 *   hold ceil(max_len / page_size) pages.  page_size must be a multiple of 32.
 */
int nq_attn_decode_paged_fwd(const void* q, const int64_t* q_strides, const void* k_new,
                             const int64_t* k_new_strides, const void* v_new,
                             const int64_t* v_new_strides, const float* k_weight, void* k_pool,
                             const int64_t* k_pool_strides, void* v_pool,
                             const int64_t* v_pool_strides, const int32_t* block_table,
                             int64_t bt_stride, int page_size, const int32_t* lens,
                             int32_t* lens_out, void* o, const int64_t* o_strides, void* workspace,
                             int64_t workspace_bytes, int B, int Hq, int Hkv, int D, int max_len,
                             int chunk, int dtype, const float* q_weight, float eps,
                             const float* cos_tab, const float* sin_tab, int max_pos,
                             const int32_t* q_pos, int q_pos0, float sm_scale, void* stream);

/*
 * nq_attn_decode_paged_fwd without a workspace argument, allocating nothing.
 * It has no counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  The workspace is a static device array
 * of NQ_DECODE_SCRATCH_BYTES that each GPU the library runs on holds until
 * the process ends; sizes whose workspace
 * (nq_attn_decode_workspace_bytes) exceeds it are refused with
 * NQ_ERR_WORKSPACE (fp32 caches use no workspace and are never refused for
 * it).  The caller still passes every input and output.  All
 * calls on one GPU share that GPU's array: calls that overlap on one GPU (on
 * different streams, or from different threads) race.  Results are those of
 * nq_attn_decode_paged_fwd with the same arguments.
 */
#define NQ_DECODE_SCRATCH_BYTES (16ll << 20)
int nq_attn_decode_paged_fwd_noalloc(const void* q, const int64_t* q_strides, const void* k_new,
                                     const int64_t* k_new_strides, const void* v_new,
                                     const int64_t* v_new_strides, const float* k_weight,
                                     void* k_pool, const int64_t* k_pool_strides, void* v_pool,
                                     const int64_t* v_pool_strides, const int32_t* block_table,
                                     int64_t bt_stride, int page_size, const int32_t* lens,
                                     int32_t* lens_out, void* o, const int64_t* o_strides, int B,
                                     int Hq, int Hkv, int D, int max_len, int chunk, int dtype,
                                     const float* q_weight, float eps, const float* cos_tab,
                                     const float* sin_tab, int max_pos, const int32_t* q_pos,
                                     int q_pos0, float sm_scale, void* stream);

/*
 * Append S rows per sequence to a paged cache: K rows QK-Normed (k_weight,
 * NULL = none) and rotated (cos_tab, NULL = none), V rows copied.  Token s of
 * sequence b becomes row row_base[b] + s (row_base NULL: row0 + s) of that
 * sequence.  Positions as in nq_qk_norm_rope (pos, pos_base, pos0).  k or v
 * may be NULL to append only the other.  The paged form of the K/V jobs of
 * nq_qk_norm_rope (model/attention.py:31-38 and :95-103).
 */
int nq_kv_append_paged(const void* k, const int64_t* k_strides, const void* v,
                       const int64_t* v_strides, void* k_pool, const int64_t* k_pool_strides,
                       void* v_pool, const int64_t* v_pool_strides, const int32_t* block_table,
                       int64_t bt_stride, int page_size, int B, int S, int Hkv, int D,
                       int dtype_in, int dtype_out, const float* k_weight, float eps,
                       const float* cos_tab, const float* sin_tab, int max_pos,
                       const int32_t* pos, const int32_t* pos_base, int pos0,
                       const int32_t* row_base, int row0, void* stream);

/*
 * Merge an attention partial into an accumulator, both computed over disjoint
 * key sets: the online-softmax combine of ring attention
 * (distributed/context_parallel.py:120-127 and 133-134), done with each
 * part's log-sum-exp.
 *
 * o / o_part: (B, H, S, D) normalised outputs with strides {batch, head, seq};
 * lse / lse_part: fp32 (B, H, S) contiguous natural-log sum-exp of the scaled
 *   scores (as nq_attn_prefill_fwd writes), -inf for a row with no keys.
 * On return lse = log(exp(lse) + exp(lse_part)) and
 *   o = o * exp(lse_old - lse) + o_part * exp(lse_part - lse); a row empty in
 *   both stays empty (o = 0, lse = -inf).
 */
int nq_attn_merge(void* o, const int64_t* o_strides, float* lse, const void* o_part,
                  const int64_t* part_strides, const float* lse_part, int B, int H, int S, int D,
                  int dtype, void* stream);

/*
 * Bytes of fp32 workspace nq_attn_bwd needs: per query row, the forward's LSE
 * (in log2 units) and Delta = rowsum(dO * O), both formed by its first kernel
 * and read by its second.
 */
int64_t nq_attn_bwd_workspace_bytes(int B, int Hq, int S);

/*
 * Attention backward (FlashAttention-2 with the forward's LSE): the gradient
 * of F.scaled_dot_product_attention (model/attention.py:110-115) that
 * training's loss.backward() runs today, for GQA without the
 * repeat_interleave (the kv-head gradients are summed over their G query
 * heads).
 *
 * q, k, v: the forward's operands as the attention saw them (Q-hat and K-hat,
 *   i.e. after QK-Norm and RoPE), (B, H, S|T, D) with strides {batch, head,
 *   seq}; o, dout: (B, Hq, S, D) forward output and its gradient; lse: fp32
 *   (B, Hq, S) from nq_attn_prefill_fwd (same q, k, v, causal and sm_scale).
 * dq (B, Hq, S, D), dk / dv (B, Hkv, T, D): outputs, fully written.
 * causal keeps key j for query i iff j <= i + T - S (needs S <= T).
 * key_lens: optional int32 (B), as in nq_attn_prefill_fwd (the forward's
 *   key padding): keys at or past key_lens[b] get zero dK / dV.
 * workspace: nq_attn_bwd_workspace_bytes(B, Hq, S) bytes.
 * Requires 128 % (Hq / Hkv) == 0.  Storage dtype bf16 (products on bf16
 * MFMA) or fp32 (products on fp32 MFMA, as the reference's fp32 autograd);
 * accumulation and softmax in fp32 either way.
 */
int nq_attn_bwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                const void* v, const int64_t* v_strides, const void* o, const int64_t* o_strides,
                const void* dout, const int64_t* do_strides, const float* lse,
                const int32_t* key_lens, void* dq, const int64_t* dq_strides, void* dk,
                const int64_t* dk_strides, void* dv,
                const int64_t* dv_strides, void* workspace, int64_t workspace_bytes, int B, int Hq,
                int Hkv, int S, int T, int D, int dtype, int causal, float sm_scale, void* stream);

/*
 * nq_attn_bwd of a forward that ran with an attention bias
 * (nq_attn_prefill_bias_fwd): bias as there, plus its transpose bias_t
 * (bias_t[b, h, j, i] at bias_t + b * bias_t_strides[0] +
 * h * bias_t_strides[1] + j * bias_t_strides[2] + i, each key's queries
 * contiguous and readable up to S rounded up to 8; same alignment rules),
 * which the dK/dV kernel reads.  lse is the bias forward's (-inf rows get
 * zero gradients).  Other arguments as nq_attn_bwd.
 */
int nq_attn_bwd_bias(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                     const void* v, const int64_t* v_strides, const void* o, const int64_t* o_strides,
                     const void* dout, const int64_t* do_strides, const float* lse,
                     const int32_t* key_lens, const void* bias, const int64_t* bias_strides,
                     const void* bias_t, const int64_t* bias_t_strides, void* dq,
                     const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                     const int64_t* dv_strides, void* workspace, int64_t workspace_bytes, int B, int Hq,
                     int Hkv, int S, int T, int D, int dtype, int causal, float sm_scale,
                     void* stream);

/*
 * Bytes of fp32 workspace nq_qk_norm_rope_bwd needs when it forms the weight
 * gradient: one partial sum of D values per block of its grid.
 */
int64_t nq_qk_norm_rope_bwd_workspace_bytes(int B, int S, int H, int D);

/*
 * Backward of QK-Norm + RoPE (model/norm.py:17-22 and model/rope.py:133-161
 * as applied at attention.py:95-100): given the pre-norm rows x and the
 * gradient dy of y = rope(rmsnorm(x) * weight), writes dx and the weight
 * gradient dweight (fp32, D elements, fully written).  The blocks store
 * partial sums of dweight in the workspace
 * (nq_qk_norm_rope_bwd_workspace_bytes), which a second launch adds in block
 * order: dweight is the same bit for bit on every run.  weight / dweight
 * NULL: no norm (workspace unused); cos_tab NULL: no rotation.  Positions as
 * in nq_qk_norm_rope.  x, dy, dx: (B, H, S, D) with strides {batch, head,
 * seq}.
 */
int nq_qk_norm_rope_bwd(const void* x, const int64_t* x_strides, const void* dy,
                        const int64_t* dy_strides, void* dx, const int64_t* dx_strides,
                        const float* weight, float* dweight, void* workspace, int64_t workspace_bytes,
                        int B, int S, int H, int D, int dtype, float eps, const float* cos_tab,
                        const float* sin_tab, int max_pos, const int32_t* pos, const int32_t* pos_base,
                        int pos0, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NQ_ATTN_H_ */
