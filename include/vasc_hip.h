/*
 * vasc_hip.h -- C-ABI of the MI355X (gfx950) sparse global-attention path.
 *
 * Plain pointers, 64-bit sizes and element strides, an explicit HIP stream
 * (passed as void*, NULL = the legacy default stream) and an int status.
 * No entry point allocates device memory: scratch comes from a caller
 * buffer sized by the matching *_workspace_size query. Entry points are
 * safe to call from any host thread on distinct streams; the only mutable
 * global is the thread-local error string returned by vasc_last_error().
 *
 * Tensors are bfloat16 (passed as uint16_t bit patterns) unless noted.
 * "[B,H,T,D] strided" means element (b,h,t,d) lives at
 *   ptr[b*stride_b + h*stride_h + t*stride_t + d]   (d is contiguous).
 *
 * Reference interfaces replaced (paths relative to /root/reference; ZIP: is
 * a member of third_party/spargeattn.zip under spargeattn/):
 *   predict_attention ........ src/sparse_vggt/models/attention.py:31-104
 *   _mean_pool_contiguous_value_blocks ... src/sparse_vggt/utils/sparse_wrapper.py:2839-2861
 *   get_block_mask ........... sparse_wrapper.py:1199-1268
 *   get_cosa_value_risk_pair_debt_mask ... sparse_wrapper.py:3632-4098
 *   block_map_lut_triton ..... ZIP:spas_sage_attn/utils.py:54-87
 *   _qattn.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf[_with_pv_threshold]
 *                              ZIP:csrc/qattn/attn_cuda.h:19-45, pybind.cpp:5-13
 */
#ifndef VASC_HIP_H
#define VASC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VASC_OK 0
#define VASC_ERR_ARGUMENT 1    /* invalid pointer, size or stride          */
#define VASC_ERR_UNSUPPORTED 2 /* valid request outside the built variants */
#define VASC_ERR_HIP 3         /* a HIP runtime call failed                */

#define VASC_MODE_TOPK 0
#define VASC_MODE_VASC 1

/* Message of the last non-zero status returned on the calling thread. */
const char *vasc_last_error(void);

/* ABI revision of this header (bumped on any signature change). */
int vasc_abi_version(void);

/*
 * Kernel 1a: block mean pooling (avg_pool1d ceil_mode semantics: the tail
 * block averages its real tokens) of Q over block_q tokens and of K and V
 * over block_k tokens, each mean rounded to bfloat16 as the reference does
 * under bf16 autocast, plus the pair innovation of the pooled V
 * (0.5*sqrt(mean_d (V[2p]-V[2p+1])^2), sparse_wrapper.py:3733-3740).
 * Replaces the pooling of predict_attention (attention.py:60-68) and
 * _mean_pool_contiguous_value_blocks (sparse_wrapper.py:2839-2861).
 * Any of q/k/v may be NULL to skip it (innovation needs v).
 * Outputs are contiguous: pooled_q [B,H,ceil(nq/block_q),d],
 * pooled_k / pooled_v [B,H,ceil(nk/block_k),d], innovation
 * [B,H,ceil(ceil(nk/block_k)/2)] float32.
 * Built variant: d == 64, block_q == 128, block_k == 64.
 */
int vasc_pool_qkv(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                  const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                  const uint16_t *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                  int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t d,
                  int64_t block_q, int64_t block_k,
                  uint16_t *pooled_q, uint16_t *pooled_k, uint16_t *pooled_v,
                  float *innovation, void *stream);

/*
 * predict_attention's pooling with pool_mode="max" (attention.py:31-104,
 * F.max_pool1d with ceil_mode): per-feature max of Q over 128-token blocks and
 * of K over 64-token blocks, bf16 (exact). Same layout rules as
 * vasc_pool_qkv; V and the innovation stay on the mean path.
 */
int vasc_pool_qk_max(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                     const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                     int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t d,
                     int64_t block_q, int64_t block_k, uint16_t *pooled_q,
                     uint16_t *pooled_k, void *stream);

/*
 * Kernel 1b: pooled attention probabilities
 *   prob = softmax_k( bf16( bf16(pooled_q . pooled_k) * scale ) )  (fp32)
 * i.e. the score/softmax of predict_attention (attention.py:97-101) with the
 * roundings of its bf16 autocast matmul. round_bf16 = 0 skips both
 * bfloat16 roundings. pooled_q [B,H,qb,d], pooled_k [B,H,kb,d] contiguous;
 * prob [B,H,qb,kb] float32 contiguous; scale finite and > 0. priority:
 * NULL, or a second [B,H,qb,kb] output receiving max(prob, 0) with NaN -> 0,
 * the VASC ledger's QK-order priority (sparse_wrapper.py:3680-3684, 4030).
 * kb <= 1280: one launch (a workgroup holds 32 query rows against every
 * key in registers) and no workspace (NULL allowed). Larger kb: workspace
 * of at least vasc_pooled_softmax_workspace_size(B, H, qb, kb) bytes, 8-byte
 * aligned (per-row softmax states of each 256-key block, written by a first
 * kernel and merged by the second; no state is kept between calls).
 * Built variant: d == 64; kb < 2^22.
 */
int vasc_pooled_softmax(const uint16_t *pooled_q, const uint16_t *pooled_k,
                        int64_t B, int64_t H, int64_t qb, int64_t kb, int64_t d,
                        float scale, int32_t round_bf16, float *prob,
                        float *priority, void *workspace, void *stream);

/* Bytes of the vasc_pooled_softmax workspace (B*H*ceil(kb/256)*qb*8); 0 for
 * empty shapes and for kb <= 1280 (no workspace). Host-only. */
int64_t vasc_pooled_softmax_workspace_size(int64_t B, int64_t H, int64_t qb, int64_t kb);

/*
 * Pair innovation of given float32 pooled values [B,H,kb,d] (contiguous),
 * bit-identical to the innovation written by vasc_pool_qkv for the same
 * pooled values (sparse_wrapper.py:3733-3740). NaN -> 0, +-inf -> +-FLT_MAX
 * first (sparse_wrapper.py:3690-3694). Built variant: d == 64.
 */
int vasc_pair_innovation(const float *pooled_v, int64_t B, int64_t H,
                         int64_t kb, int64_t d, float *innovation,
                         void *stream);

/* Bytes of workspace vasc_select_blocks needs for these sizes. */
size_t vasc_select_workspace_size(int64_t B, int64_t H, int64_t q_blocks,
                                  int64_t k_blocks);

/* Regions of the VASC selection workspace that hold per-call results after
 * a VASC_MODE_VASC call (read back for the reference's routing statistics,
 * sparse_wrapper.py:4032-4096): */
#define VASC_WS_ROW_TOTAL 0     /* [B,H,Q] f32: sum_k score*innovation (risk total) */
#define VASC_WS_ROW_PAIR_SUM 1  /* [B,H,Q] f32: sum_p of the row's pair arrival   */
#define VASC_WS_ROW_CAPACITY 2  /* [B,H,Q] i32: the row's QK capacity             */
#define VASC_WS_ADMITTED_DEBT 3 /* [B,H,P] f32: admitted debt per pair            */

/* Byte offset of a region inside the workspace for these sizes; -1 for an
 * unknown region or empty sizes. Host-only. */
int64_t vasc_select_workspace_offset(int64_t B, int64_t H, int64_t q_blocks,
                                     int64_t k_blocks, int32_t region);

/*
 * Kernel 2: per-row block selection writing ascending index lists.
 *
 * mode VASC_MODE_TOPK: get_block_mask top-k (sparse_wrapper.py:1199-1268)
 *   keeping the max(topk,1) largest scores per row, ties to the lower index.
 * mode VASC_MODE_VASC: get_cosa_value_risk_pair_debt_mask
 *   (sparse_wrapper.py:3632-4098) in the release configuration, including
 *   the ledger settlement of the previous layer, the global service gate,
 *   conservative arrival/debt projection, and the QK-admission service for
 *   the next layer.
 *
 * score       [B,H,Q,K] float32 contiguous pooled probabilities.
 * innovation  [B,H,ceil(K/2)] float32 (VASC only).
 * topk        base budget int(K*(1-s)); the fill rule raises 0 to 1.
 * row_cap     optional [B,H,Q] int32 per-row budget; NULL derives it from
 *             topk (and, in VASC, force_last) as block_sparse_attn_cuda does.
 *             TOPK: the per-row count (cdf threshold, vasc_cdf_counts), the
 *             forced tail added on top, each at most max_capacity (0 = K).
 *             VASC: the row's QK capacity (base count including the tail).
 * protected_mask optional [B,H,Q,K] uint8 (VASC): priority FLT_MAX.
 * force_last  mixed tail block K-1: kept in TOPK, protected in VASC and
 *             counted in the derived capacity (sparse_wrapper.py:7599-7662).
 * max_capacity M (VASC): at most M blocks per row (the capacity hint);
 *             TOPK with row_cap: the largest row_cap entry (0 = K).
 * sink_blocks trailing always-on blocks K..K+sink-1 appended to each list.
 * debt_in, pending_arrival, prev_service [B,H,P] float32, each may be NULL
 *             (NULL pending = no previous layer to settle).
 * debt_out, arrival_out, service_out [B,H,P] float32 (VASC, required),
 *             each disjoint from the three inputs and from each other: the
 *             ledger cannot be updated in place (one head's inputs are read
 *             by every workgroup of the head while others write its
 *             outputs). Overlapping ranges are rejected (VASC_ERR_ARGUMENT).
 * gate_out    optional int32 scalar: 1 when the debt priority was used.
 * priority_out optional [B,H,Q,K] float32 execution priority.
 * mask_out    optional [B,H,Q,K] uint8 support of the patch blocks.
 * index_out   [B,H,Q,width] int32 ascending block indices: the kept patch
 *             blocks, then the sink blocks (count entries in all), then -1
 *             to the end of the row; count_out [B,H,Q] int32.
 * Built variant: K <= 8192.
 */
int vasc_select_blocks(const float *score, const float *innovation,
                       int64_t B, int64_t H, int64_t Q, int64_t K,
                       int32_t mode, int32_t topk, const int32_t *row_cap,
                       const uint8_t *protected_mask, int32_t force_last,
                       int32_t max_capacity, int32_t sink_blocks,
                       const float *debt_in, const float *pending_arrival,
                       const float *prev_service, float *debt_out,
                       float *arrival_out, float *service_out,
                       int32_t *gate_out, float *priority_out,
                       uint8_t *mask_out, int32_t *index_out, int64_t width,
                       int32_t *count_out, void *workspace,
                       size_t workspace_bytes, void *stream);

/* Largest workspace (bytes) vasc_select_blocks_noalloc can serve. */
#define VASC_SELECT_SCRATCH_BYTES (32u << 20)

/*
 * vasc_select_blocks without a workspace argument: it allocates nothing
 * (no hipMalloc, hipFree or allocating library call) and takes its scratch
 * from a 32 MiB array of device memory inside the library, one copy per
 * GPU, held until the process ends. No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, results
 * and errors as vasc_select_blocks; sizes whose workspace
 * (vasc_select_workspace_size) exceeds VASC_SELECT_SCRATCH_BYTES are
 * rejected with VASC_ERR_ARGUMENT (at B = 1, H = 16: up to 4096 key blocks
 * with 2048 query blocks). Every call on one GPU shares that GPU's scratch:
 * calls that overlap in time on one GPU (other streams, other threads) race
 * and must be serialised by the caller. The first call on a device resolves
 * the scratch address with that device current.
 */
int vasc_select_blocks_noalloc(const float *score, const float *innovation,
                               int64_t B, int64_t H, int64_t Q, int64_t K,
                               int32_t mode, int32_t topk,
                               const int32_t *row_cap,
                               const uint8_t *protected_mask,
                               int32_t force_last, int32_t max_capacity,
                               int32_t sink_blocks, const float *debt_in,
                               const float *pending_arrival,
                               const float *prev_service, float *debt_out,
                               float *arrival_out, float *service_out,
                               int32_t *gate_out, float *priority_out,
                               uint8_t *mask_out, int32_t *index_out,
                               int64_t width, int32_t *count_out,
                               void *stream);

/*
 * Terminal ledger settlement (finalize_cosa_value_risk_pair_debt,
 * sparse_wrapper.py:4101-4177): debt_out = max(debt_in + pending - service, 0)
 * elementwise over n floats; debt_in may be NULL (zeros).
 */
int vasc_settle_terminal(const float *debt_in, const float *pending_arrival,
                         const float *service, int64_t n, float *debt_out,
                         void *stream);

/*
 * Per-row counts of get_block_mask's cdf-threshold branch
 * (sparse_wrapper.py:1238-1254; fill rule ZIP:spas_sage_attn/utils.py:289).
 * Replaces the torch.sort + torch.cumsum + torch.searchsorted sequence.
 *
 * score       [B,H,Q,K] float32 contiguous pooled probabilities.
 * thresholds  [H] float32 device array T_h = f32(thr_h + eps).
 * count_out   [B,H,Q] int32: length of the prefix of the descending row
 *             whose sequential float32 running sum stays <= T_h, raised to
 *             min_count (the ratio budget when a ratio is also given), and
 *             at least 1.
 * base_out    optional [B,H,Q] int32: count plus the forced mixed tail
 *             (force_last and block K-1 not among the first `count`), the
 *             row capacity the VASC selector takes.
 * Built variant: K <= 8192.
 */
int vasc_cdf_counts(const float *score, int64_t B, int64_t H, int64_t Q,
                    int64_t K, const float *thresholds, int32_t min_count,
                    int32_t force_last, int32_t *count_out, int32_t *base_out,
                    void *stream);

/*
 * The VASC selector's selected indices: per row, the M blocks of largest
 * priority, largest first, equal priorities in ascending block index.
 * Replaces priority.topk(M, dim=-1, sorted=True).indices
 * (sparse_wrapper.py:3887-3894), stored as routing_state
 * "cosa_value_risk_pair_selected_indices" (sparse_wrapper.py:4024-4026).
 *
 * priority   [rows,K] float32 contiguous (vasc_select_blocks' priority_out).
 * index      optional [rows,width] int32: vasc_select_blocks' index lists
 *            of a selection that kept each row's largest priorities under
 *            the same tie rule (the VASC selection that wrote `priority`;
 *            count: their counts, sink: the sink blocks appended to each
 *            list). A row that kept exactly M patch blocks takes them from
 *            its list instead of ranking the row.
 * order_out  [rows,M] int64.
 * 0 <= M <= K (M == 0 writes nothing); width >= M + sink when index is
 * given. Built variant: K <= 8192.
 */
int vasc_priority_order(const float *priority, const int32_t *index,
                        const int32_t *count, int64_t width, int32_t sink,
                        int64_t rows, int64_t K, int64_t M, int64_t *order_out,
                        void *stream);

/* Elements (bf16) of the packed V buffer for these sizes. */
int64_t vasc_packed_v_elems(int64_t B, int64_t H, int64_t nk, int64_t d);

/*
 * Kernel 3: pack V [B,H,nk,d] (strided) into per-64-key-block transposed
 * tiles vt [B,H,ceil(nk/64),d,64] (contiguous), keys permuted into the
 * MFMA operand order of the attention kernel and zero padded past nk.
 * Precedent: SpargeAttn's TransposePadPermuteKernel (ZIP:csrc/fused/fused.cu:26-78).
 * Built variant: d == 64.
 */
int vasc_pack_v(const uint16_t *v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                int64_t B, int64_t H, int64_t nk, int64_t d, uint16_t *vt,
                void *stream);

/*
 * Kernel 4: block-sparse flash attention forward, bf16 QK^T and PV on MFMA,
 * fp32 online softmax. Query block i (128 rows) attends to the 64-key blocks
 * listed in block_index[b,h,i,0:block_count[b,h,i]]; keys >= nk are masked.
 * index_is_delta = 0: absolute ascending indices (vasc_select_blocks);
 * index_is_delta = 1: SpargeAttn's delta LUT (first entry absolute).
 * Out-of-range blocks are skipped; rows with count 0 are written as zeros.
 * Replaces _qattn.qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf
 * (ZIP:csrc/qattn/attn_cuda.h:19-32) with bf16 inputs instead of int8 +
 * scales. q, o [B,H,nq,d] strided; k [B,H,nk,d] strided; vt from
 * vasc_pack_v. Built variant: d == 64.
 */
int vasc_block_sparse_attn_fwd(const uint16_t *q, int64_t q_sb, int64_t q_sh,
                               int64_t q_st, const uint16_t *k, int64_t k_sb,
                               int64_t k_sh, int64_t k_st, const uint16_t *vt,
                               uint16_t *o, int64_t o_sb, int64_t o_sh,
                               int64_t o_st, int64_t B, int64_t H, int64_t nq,
                               int64_t nk, int64_t d,
                               const int32_t *block_index, int64_t index_width,
                               const int32_t *block_count,
                               int32_t index_is_delta, float sm_scale,
                               void *stream);

/*
 * vasc_block_sparse_attn_fwd with the PV post-cut of the reference's
 * qk_int8_sv_f16_accum_f16_block_sparse_attn_inst_buf_with_pv_threshold
 * (ZIP:csrc/qattn/qk_int_sv_f16_cuda_sm80.cu:188-376, per-block mode;
 * skip branch qk_int_sv_f16_cuda_sm80.cuh:291-381, update_mo
 * attn_utils.cuh:419-466) and its return_pv_count map. Per 128-row query
 * block and listed key block: gap = max over rows of (block row max -
 * running row max), log2 units (logit * sm_scale * log2 e); the running max
 * starts at -5e6 and follows every listed block; the block's exp, row sum and
 * PV run only when gap + pv_threshold[h] > 0.
 *
 * pv_threshold  [H] float32 device array (log2 units).
 * pv_map        optional [B,H,ceil(nq/128)*4,ceil(nk/64)] int32, zeroed by
 *               the caller: 1 where a 32-row query wave ran a block's PV.
 */
int vasc_block_sparse_attn_pv_fwd(const uint16_t *q, int64_t q_sb, int64_t q_sh,
                                  int64_t q_st, const uint16_t *k, int64_t k_sb,
                                  int64_t k_sh, int64_t k_st, const uint16_t *vt,
                                  uint16_t *o, int64_t o_sb, int64_t o_sh,
                                  int64_t o_st, int64_t B, int64_t H, int64_t nq,
                                  int64_t nk, int64_t d,
                                  const int32_t *block_index, int64_t index_width,
                                  const int32_t *block_count,
                                  int32_t index_is_delta, float sm_scale,
                                  const float *pv_threshold, int32_t *pv_map,
                                  void *stream);

/*
 * Kernel 4 for a whole global layer: the patch queries q_patch [B,H,n_patch,d]
 * attend to their listed blocks as in vasc_block_sparse_attn_fwd (absolute
 * indices), and the special-token queries q_special [B,H,n_special,d] attend
 * to every key, in the same launch (attention.py:8464-8484 runs them through
 * a separate dense SDPA). k [B,H,nk,d] and vt hold all tokens, patch tokens
 * first. Outputs o_patch [B,H,n_patch,d], o_special [B,H,n_special,d]; all
 * strided as in vasc_block_sparse_attn_fwd. n_special may be 0 (q_special,
 * o_special then unused). Built variant: d == 64.
 */
int vasc_global_attn_fwd(const uint16_t *q_patch, int64_t qp_sb, int64_t qp_sh,
                         int64_t qp_st, const uint16_t *q_special,
                         int64_t qs_sb, int64_t qs_sh, int64_t qs_st,
                         const uint16_t *k, int64_t k_sb, int64_t k_sh,
                         int64_t k_st, const uint16_t *vt, uint16_t *o_patch,
                         int64_t op_sb, int64_t op_sh, int64_t op_st,
                         uint16_t *o_special, int64_t os_sb, int64_t os_sh,
                         int64_t os_st, int64_t B, int64_t H, int64_t n_patch,
                         int64_t n_special, int64_t nk, int64_t d,
                         const int32_t *block_index, int64_t index_width,
                         const int32_t *block_count, float sm_scale,
                         void *stream);

/*
 * vasc_global_attn_fwd writing the layer's output order: the patch and
 * special query results go straight to their frame-major token rows of out
 * [B, N*P, H*d] (contiguous), the tensor the layer's restore to frame-major
 * order and transpose before the output projection produce
 * (attention.py:8992-9027, tokens.py:64-126): patch query i of frame
 * n = i / (P-S) to token n*P + S + i % (P-S), special query j to token
 * (j / S)*P + j % S. n_patch = N*(P-S), n_special = N*S, nk = N*P.
 * Built variant: d == 64.
 */
int vasc_global_attn_tokens_fwd(const uint16_t *q_patch, int64_t qp_sb,
                                int64_t qp_sh, int64_t qp_st,
                                const uint16_t *q_special, int64_t qs_sb,
                                int64_t qs_sh, int64_t qs_st,
                                const uint16_t *k, int64_t k_sb, int64_t k_sh,
                                int64_t k_st, const uint16_t *vt,
                                uint16_t *out, int64_t B, int64_t H, int64_t N,
                                int64_t P, int64_t S, int64_t nk, int64_t d,
                                const int32_t *block_index,
                                int64_t index_width,
                                const int32_t *block_count, float sm_scale,
                                void *stream);

/* Dense variant of kernel 4: every query block attends to all key blocks. */
int vasc_dense_attn_fwd(const uint16_t *q, int64_t q_sb, int64_t q_sh,
                        int64_t q_st, const uint16_t *k, int64_t k_sb,
                        int64_t k_sh, int64_t k_st, const uint16_t *vt,
                        uint16_t *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
                        int64_t B, int64_t H, int64_t nq, int64_t nk,
                        int64_t d, float sm_scale, void *stream);

/*
 * Kernel 5a: token layout of a global layer. Replaces the head split,
 * q_norm / k_norm, rotary embedding and the [patch; special] reorder of
 * attention.py:8351-8469 (tokens.py:2-62: six full copies) with one pass.
 *
 * q, k, v: frame-major tokens, T = N*P (per frame S special tokens, then
 *   P-S patch tokens), element (b,t,h,j) at ptr + b*sb + t*st + h*sh + j
 *   (j contiguous). The fused qkv projection [B,T,3*H*d] is q = qkv,
 *   k = qkv + H*d, v = qkv + 2*H*d with st = 3*H*d, sh = d.
 * q_norm / k_norm != 0: LayerNorm over the d features of each (token, head)
 *   with optional weight and bias [d] (NULL: 1 / 0) and eps, before the
 *   rotary embedding; 1: weight and bias are float32, 2: bfloat16 (the
 *   parameters of a bf16 model are read as they are, no converted copy).
 * pos != NULL: 2D rotary embedding of q and k. Token (b,t) has the integer
 *   row / column position pos[b*pos_sb + t*pos_st + 0 / 1]; features
 *   [0, d/2) rotate with the row, [d/2, d) with the column; inside a half,
 *   feature j < d/4 pairs with j + d/4:
 *     out_j      = x_j cos(a) - x_{j+d/4} sin(a)
 *     out_{j+d/4} = x_{j+d/4} cos(a) + x_j sin(a),   a = position * freq_j
 *   with cos/sin read from rope_cos / rope_sin [rope_n, d/4] (float32,
 *   entry (position, j), 16-byte aligned); positions are clamped into
 *   [0, rope_n).
 * Outputs (contiguous bf16): q_patch [B,H,N*(P-S),d], q_special [B,H,N*S,d],
 *   k_out / v_out [B,H,T,d] with the patch tokens of all frames first, then
 *   the special tokens. Arithmetic in float32, one bf16 rounding per output.
 *   v_out == NULL: v is not packed (v may then be NULL); a caller that packs
 *   V for attention straight from the projection (vasc_pack_v takes strided
 *   rows) skips writing and re-reading it.
 * Built variant: d == 64.
 */
int vasc_pack_qkv(const uint16_t *q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                  const uint16_t *k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                  const uint16_t *v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                  int64_t B, int64_t H, int64_t N, int64_t P, int64_t S,
                  int64_t d, const void *q_norm_w, const void *q_norm_b,
                  float q_eps, int32_t q_norm, const void *k_norm_w,
                  const void *k_norm_b, float k_eps, int32_t k_norm,
                  const int32_t *pos, int64_t pos_sb, int64_t pos_st,
                  const float *rope_cos, const float *rope_sin, int64_t rope_n,
                  uint16_t *q_patch, uint16_t *q_special, uint16_t *k_out,
                  uint16_t *v_out, void *stream);

/*
 * Kernel 5a + 1a + 3 fused for a global layer that pools by block means:
 * the layout of vasc_pack_qkv (same inputs, same q_patch / q_special /
 * k_out, bit for bit) together with
 *   vt          V of the [patch; special] order as vasc_pack_v's MFMA tiles
 *               [B,H,ceil(N*P/64),d,64] (V is never written in token rows);
 *   pooled_q    [B,H,ceil(Np/128),d], pooled_k / pooled_v [B,H,ceil(Np/64),d]
 *               (Np = N*(P-S)): bf16 block means of the packed patch q / k
 *               and of the patch v, tail blocks over their real tokens
 *               (predict_attention, attention.py:31-104, on q_patch and the
 *               patch keys; _mean_pool_contiguous_value_blocks,
 *               sparse_wrapper.py:2839-2861); each may be NULL;
 *   innovation  [B,H,ceil(ceil(Np/64)/2)] float32 pair innovation of the
 *               pooled V blocks (sparse_wrapper.py:3733-3740), or NULL.
 * No single reference function does this: it replaces the layout of
 * attention.py:8351-8469, the pooling of attention.py:31-104 and the value
 * pooling of sparse_wrapper.py:2839-2861 and 3733-3740 in one pass, so the
 * packed q, k and the V tiles are read again only by the attention. Pooled
 * sums are float32 in a fixed order (per thread, then the 8 row groups of a
 * wave, then the four waves), within one bf16 rounding of the exact mean.
 * Requires S < P. Built variant: d == 64.
 */
int vasc_pack_global(const uint16_t *q, int64_t q_sb, int64_t q_st, int64_t q_sh,
                     const uint16_t *k, int64_t k_sb, int64_t k_st, int64_t k_sh,
                     const uint16_t *v, int64_t v_sb, int64_t v_st, int64_t v_sh,
                     int64_t B, int64_t H, int64_t N, int64_t P, int64_t S,
                     int64_t d, const void *q_norm_w, const void *q_norm_b,
                     float q_eps, int32_t q_norm, const void *k_norm_w,
                     const void *k_norm_b, float k_eps, int32_t k_norm,
                     const int32_t *pos, int64_t pos_sb, int64_t pos_st,
                     const float *rope_cos, const float *rope_sin, int64_t rope_n,
                     uint16_t *q_patch, uint16_t *q_special, uint16_t *k_out,
                     uint16_t *vt, uint16_t *pooled_q, uint16_t *pooled_k,
                     uint16_t *pooled_v, float *innovation, void *stream);

/*
 * Kernel 5b: attention outputs in [patch; special] order back to the
 * frame-major token layout the output projection reads (attention.py:
 * 8992-9027 with tokens.py:102-126 and the transpose/reshape):
 * out[b, t, h*d + j] from x_patch [B,H,N*(P-S),d] or x_special [B,H,N*S,d]
 * (strided as (b, h, token)). out [B,N*P,H*d] contiguous bf16.
 * Built variant: d == 64.
 */
int vasc_restore_tokens(const uint16_t *x_patch, int64_t p_sb, int64_t p_sh,
                        int64_t p_st, const uint16_t *x_special, int64_t s_sb,
                        int64_t s_sh, int64_t s_st, int64_t B, int64_t H,
                        int64_t N, int64_t P, int64_t S, int64_t d,
                        uint16_t *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* VASC_HIP_H */
