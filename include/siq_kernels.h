/*
 * siq_kernels.h -- C ABI of the SiQ-VL training hot path on MI355X (gfx950).
 *
 * Five operators, all hand-written HIP behind this plain-C boundary:
 *   1. varlen (cu_seqlens-packed) flash attention, forward and backward,
 *      causal GQA (Qwen2.5 decoder) or bidirectional (SigLIP tower);
 *   2. fused lm_head linear + cross-entropy, forward and backward, without
 *      materialising the [N, V] logits;
 *   3. the rotary position embedding of q and k that precedes attention in
 *      the decoder, forward and backward, in one pass each;
 *   4. the pixel-shuffle projector (vision features to text embeddings),
 *      forward and backward, with the shuffle folded into the GEMM loads;
 *   5. the splice of the projected vision rows into the token embeddings,
 *      fused with the embedding gather, and its embedding-table gradient.
 *
 * Conventions
 *  - Every entry point returns an int status (SIQ_OK = 0, < 0 on error) and
 *    records a message readable with siq_last_error() (thread-local).
 *  - All tensors are device pointers owned by the caller.  The library never
 *    allocates, frees or keeps pointers beyond a call; scratch memory is the
 *    caller's `workspace` (size from the matching *_workspace_bytes()).
 *  - `stream` is a hipStream_t (NULL = the null stream).  Work is only
 *    enqueued: no device synchronisation and no device-to-host reads.
 *  - bf16 tensors are token-major: element (token t, head h, dim d) lives at
 *    base + t * tok_stride + h * head_stride + d (d contiguous).  Base
 *    pointers and both strides must keep 16-byte alignment (strides multiple
 *    of 8 elements).
 *  - cu_seqlens are int32 device arrays of batch+1 non-decreasing offsets with
 *    cu[0] = 0 and cu[batch] = total.  They are read on the device; values
 *    outside [0, total] are clamped there, so malformed offsets give wrong
 *    numbers for the offending sequences but never an out-of-bounds access.
 */
#ifndef SIQ_KERNELS_H
#define SIQ_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIQ_ABI_VERSION 4

enum siq_status {
  SIQ_OK = 0,
  SIQ_ERR_INVALID_ARGUMENT = -1, /* shape / dtype / value rejected before launch */
  SIQ_ERR_UNSUPPORTED = -2,      /* e.g. head_dim not in {64, 128} */
  SIQ_ERR_WORKSPACE = -3,        /* workspace missing or too small */
  SIQ_ERR_ALIGNMENT = -4,        /* pointer or stride breaks 16-byte alignment */
  SIQ_ERR_LAUNCH = -5            /* the HIP runtime rejected a launch */
};

/* Element types of the entry points that take more than one. */
#define SIQ_DTYPE_BF16 0
#define SIQ_DTYPE_FP32 1

/* Version of this ABI (SIQ_ABI_VERSION of the library that was built). */
int siq_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* siq_last_error(void);

/* ---------------------------------------------------------------------------
 * Varlen attention.
 *
 * Replaces, for one packed batch, the attention call the reference reaches at
 * transformers integrations/sdpa_attention.py:154-163 (F.scaled_dot_product_
 * attention on a padded batch, reached from models/qwen2/modeling_qwen2.py:
 * 216-230 and models/siglip/modeling_siglip.py:288-300) with the varlen
 * contract of modeling_flash_attention_utils.py:796-822
 * (q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
 * softmax_scale, causal).
 *
 * Shapes: q [total_q, hq, d], k/v [total_k, hkv, d], o like q, all bf16;
 * lse fp32 [hq, total_q] (natural log, contiguous); hq % hkv == 0 and q-head h
 * reads kv-head h / (hq / hkv); d in {64, 128}.  Causal masking is aligned
 * bottom-right (q row i of a sequence sees k rows <= i + len_k - len_q), which
 * is the usual top-left causal mask when len_q == len_k.
 *
 * strides[8] = {q_tok, q_head, k_tok, k_head, v_tok, v_head, o_tok, o_head}
 * (in elements).
 * ------------------------------------------------------------------------- */
size_t siq_attn_fwd_workspace_bytes(int batch, int64_t total_q, int64_t total_k, int hq, int hkv, int d);

int siq_attn_varlen_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch,
                        int max_seqlen_q, int max_seqlen_k, int64_t total_q, int64_t total_k, int hq, int hkv,
                        int d, const int64_t* strides, float softmax_scale, int causal, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Backward of siq_attn_varlen_fwd (the autograd backward of the same call in
 * the reference path).  Inputs q, k, v, o, lse as produced/consumed by the
 * forward, dout like o; outputs dq like q, dk/dv like k/v, each written in full
 * (no accumulation).
 * deterministic != 0: no atomics, bitwise reproducible (dQ in a kernel of its
 * own that recomputes S and dP).  deterministic == 0: dQ = dS K is formed in
 * the dK/dV kernel and summed with fp32 atomics in the workspace (the sum
 * order varies from run to run; the workspace grows by total_q * hq * d * 4
 * bytes; on MI355X it measured 2-3x slower than the deterministic backward at
 * the SiQ-VL shapes).  flash-attn's flash_attn_varlen_func(deterministic=...)
 * flag.
 * strides[16] = {q_tok, q_head, k_tok, k_head, v_tok, v_head, o_tok, o_head,
 *                do_tok, do_head, dq_tok, dq_head, dk_tok, dk_head, dv_tok, dv_head}. */
size_t siq_attn_bwd_workspace_bytes(int batch, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                                    int deterministic);

int siq_attn_varlen_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse,
                        const void* dout, void* dq, void* dk, void* dv, const int32_t* cu_seqlens_q,
                        const int32_t* cu_seqlens_k, int batch, int max_seqlen_q, int max_seqlen_k,
                        int64_t total_q, int64_t total_k, int hq, int hkv, int d, const int64_t* strides,
                        float softmax_scale, int causal, int deterministic, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Allocation-free siq_attn_varlen_fwd.  No counterpart in the reference: it
 * exists for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation) and takes
 * no workspace.  Same arguments (minus the workspace), validation and output,
 * bitwise, as siq_attn_varlen_fwd.  The batch's plan goes to a static device
 * array of 1 MiB per GPU (held until the process ends): batch and total_q
 * must satisfy 256 + 16 batch + 32 (total_q / 128 + batch + 1) <= 1 MiB (each
 * term rounded up to 256 bytes), e.g. batch <= 8192 with total_q <= 2^20;
 * larger calls return SIQ_ERR_WORKSPACE before anything is launched.  All
 * calls on one GPU share the array: calls that overlap on one GPU (from
 * different streams or threads) race. */
int siq_attn_varlen_fwd_noalloc(const void* q, const void* k, const void* v, void* o, float* lse,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch,
                                int max_seqlen_q, int max_seqlen_k, int64_t total_q, int64_t total_k, int hq,
                                int hkv, int d, const int64_t* strides, float softmax_scale, int causal,
                                void* stream);

/* ---------------------------------------------------------------------------
 * Attention plans: the schedule of one packed batch, built once and reused.
 *
 * The reference forwards the same cu_seq_lens_* kwargs to every decoder layer
 * (siq_vl/model/modeling.py:278-288 -> transformers modeling_qwen2.py:216-230),
 * so the work lists siq_attn_varlen_fwd / _bwd build on every call (sequence
 * extents, q tiles and dK/dV work items ordered by decreasing work) are the
 * same for all layers.  siq_attn_build_plan writes them once into `plan`
 * (siq_attn_plan_bytes, device memory owned by the caller); the *_plan entry
 * points then run the forward / backward of any layer over it.  A plan
 * depends on the offsets, total_q / total_k, hq / hkv and causal only; it
 * records them, and a kernel handed a plan built for other values writes
 * nothing and sets a mismatch bit in the plan (bytes 48..51, int32) instead of
 * touching memory outside its tensors.  Bytes 40..47 hold the scheduler's
 * overflow bits (0 by construction).
 * ------------------------------------------------------------------------- */
size_t siq_attn_plan_bytes(int batch, int64_t total_q, int64_t total_k);

int siq_attn_build_plan(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int batch, int64_t total_q,
                        int64_t total_k, int hq, int hkv, int causal, void* plan, size_t plan_bytes, void* stream);

/* siq_attn_varlen_fwd over a built plan (no workspace). */
int siq_attn_varlen_fwd_plan(const void* q, const void* k, const void* v, void* o, float* lse, int batch,
                             int64_t total_q, int64_t total_k, int hq, int hkv, int d, const int64_t* strides,
                             float softmax_scale, int causal, const void* plan, size_t plan_bytes, void* stream);

/* siq_attn_varlen_bwd over a built plan; the workspace holds the backward's
 * own scratch only (siq_attn_bwd_plan_workspace_bytes, for the same
 * deterministic flag). */
size_t siq_attn_bwd_plan_workspace_bytes(int batch, int64_t total_q, int64_t total_k, int hq, int hkv, int d,
                                         int deterministic);

int siq_attn_varlen_bwd_plan(const void* q, const void* k, const void* v, const void* o, const float* lse,
                             const void* dout, void* dq, void* dk, void* dv, int batch, int64_t total_q,
                             int64_t total_k, int hq, int hkv, int d, const int64_t* strides, float softmax_scale,
                             int causal, int deterministic, const void* plan, size_t plan_bytes, void* workspace,
                             size_t workspace_bytes, void* stream);

/* Varlen attention with the decoder's rotary embedding of q fused in.
 *
 * Replaces apply_rotary_pos_emb's q half (transformers modeling_qwen2.py:
 * 105-135, called at :206-211) together with the attention call after it:
 * siq_attn_rope_fwd_plan reads q BEFORE rotation, rotates it in registers with
 * the cos / sin rows of each token (bitwise siq_rope_fwd's q_embed), attends
 * as siq_attn_varlen_fwd_plan does (k already rotated, e.g. by siq_rope_fwd
 * with hq = 0) and writes the rotated q to q_embed for the backward.
 * siq_attn_rope_bwd_plan takes that q_embed and writes dq with respect to the
 * q BEFORE rotation (bitwise siq_rope_bwd applied to siq_attn_varlen_bwd_plan's
 * dq); dk, dv are those of siq_attn_varlen_bwd_plan (dk with respect to the
 * rotated k).  The backward is the deterministic one (its workspace:
 * siq_attn_bwd_plan_workspace_bytes(..., 1)): the rotation's backward runs in
 * the epilogue of its dQ kernel.  cos / sin: [total_q, d] bf16 rows, one per
 * packed token.
 * strides: fwd[12] = the 8 of siq_attn_varlen_fwd, q_embed (tok, head),
 * cos_tok, sin_tok; bwd[18] = the 16 of siq_attn_varlen_bwd (q = q_embed),
 * cos_tok, sin_tok. */
int siq_attn_rope_fwd_plan(const void* q, const void* k, const void* v, void* o, float* lse, void* q_embed,
                           const void* cos, const void* sin, int batch, int64_t total_q, int64_t total_k, int hq,
                           int hkv, int d, const int64_t* strides, float softmax_scale, int causal, const void* plan,
                           size_t plan_bytes, void* stream);

int siq_attn_rope_bwd_plan(const void* q_embed, const void* k, const void* v, const void* o, const float* lse,
                           const void* dout, void* dq, void* dk, void* dv, const void* cos, const void* sin, int batch,
                           int64_t total_q, int64_t total_k, int hq, int hkv, int d, const int64_t* strides,
                           float softmax_scale, int causal, const void* plan, size_t plan_bytes, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Fused linear cross-entropy (lm_head + loss), forward and backward.
 *
 * Replaces logits = lm_head(h) (transformers models/qwen2/modeling_qwen2.py:
 * 465) followed by ForCausalLMLoss / fixed_cross_entropy (loss/loss_utils.py:
 * 32-71: fp32 upcast, F.cross_entropy with ignore_index) and their autograd
 * backward.  hidden [n, hdim] bf16 row-major, weight [vocab, hdim] bf16
 * row-major, labels [n] int64 (already shifted; ignore_index rows are skipped;
 * any other value outside [0, vocab) is treated as ignored and counted in
 * *bad_labels, which the host raises on as F.cross_entropy would).
 *
 * reduction 0 ("mean"): loss = sum_valid(lse - z_y) / count_valid.
 * reduction 1 ("sum" then divide, as with num_items_in_batch):
 *   loss = sum_valid(lse - z_y) / *divisor, divisor a device fp32 scalar.
 * Outputs (device): *loss fp32 scalar, *count int64 number of valid rows,
 * dhidden [n, hdim] bf16 = d loss / d hidden, dweight [vocab, hdim] bf16 =
 * d loss / d weight (may be NULL to skip it).  Ignored rows get dhidden
 * exactly 0.
 *
 * The logits are produced chunk_tokens rows at a time: only the softmax
 * numerators of one chunk (chunk_tokens x vocab bf16, each relative to the max
 * of its 256-column tile) ever exist, in the workspace; chunks count rows
 * whose label counts (ignored rows are compacted away first).  Over two
 * chunks dweight is summed in dweight itself (the first chunk's sum rounded to
 * bf16 once); over more it is summed in an fp32 [vocab, hdim] workspace
 * buffer, which the workspace holds whenever n exceeds two chunks.
 * ------------------------------------------------------------------------- */
size_t siq_flce_workspace_bytes(int64_t n, int64_t hdim, int64_t vocab, int64_t chunk_tokens, int need_dweight);

int siq_flce_fwd_bwd(const void* hidden, const void* weight, const int64_t* labels, int64_t n, int64_t hdim,
                     int64_t vocab, int64_t ignore_index, int reduction, const float* divisor, float* loss,
                     int64_t* count, int64_t* bad_labels, void* dhidden, void* dweight, int64_t chunk_tokens,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Loss only: the same loss, count and bad_labels as siq_flce_fwd_bwd on the
 * same inputs (bitwise), without the gradient work -- the reference's
 * evaluation pass (scripts/train.py:693-699 evaluates eval_loss under
 * torch.no_grad through the same lm_head + ForCausalLMLoss call).  Only the
 * logits GEMM and the chunked logsumexp run; no softmax numerators are
 * stored.  Workspace: siq_flce_loss_workspace_bytes. */
size_t siq_flce_loss_workspace_bytes(int64_t n, int64_t hdim, int64_t vocab);

int siq_flce_loss(const void* hidden, const void* weight, const int64_t* labels, int64_t n, int64_t hdim,
                  int64_t vocab, int64_t ignore_index, int reduction, const float* divisor, float* loss,
                  int64_t* count, int64_t* bad_labels, void* workspace, size_t workspace_bytes, void* stream);

/* dst = src * (*scalar) over numel bf16 elements, rounded once from fp32
 * (a device fp32 scalar, read on the device): applies the upstream gradient
 * of the scalar loss to dhidden / dweight.  Companion of siq_flce_fwd_bwd; no
 * reference counterpart (autograd's chain rule).  src == dst scales in place
 * (and then an exact 1.0 writes nothing); any other overlap is undefined. */
int siq_scale_bf16(const void* src, void* dst, int64_t numel, const float* scalar, void* stream);

/* siq_scale_bf16(data, data, numel, scalar, stream). */
int siq_scale_bf16_inplace(void* data, int64_t numel, const float* scalar, void* stream);

/* ---------------------------------------------------------------------------
 * Rotary position embedding of q and k (Qwen2 decoder).
 *
 * Replaces apply_rotary_pos_emb (transformers models/qwen2/modeling_qwen2.py:
 * 105-135, with rotate_half; called from Qwen2Attention.forward at :206-211):
 *   q_embed = q * cos + rotate_half(q) * sin,  k_embed likewise,
 * rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2]), evaluated with the
 * reference's bf16 rounding after every op, so the results are bitwise those
 * of the reference's torch ops on the same bf16 inputs.  siq_rope_bwd applies
 * the reference's autograd of the same ops to the upstream gradients
 * (dq_embed, dk_embed) and writes dq, dk.
 *
 * Tensors are bf16 [batch, seqlen, heads, head_dim] (cos, sin:
 * [batch, seqlen, head_dim]) with element strides, head_dim contiguous:
 * strides[16] = q (b, s, h), k (b, s, h), cos (b, s), sin (b, s),
 * q_embed (b, s, h), k_embed (b, s, h) -- for siq_rope_bwd read dq_embed,
 * dk_embed, cos, sin, dq, dk.  Strides are multiples of 8 elements and base
 * pointers 16-byte aligned.  An output may be its input (same pointer and
 * strides, in place); any other overlap is undefined.  head_dim: a multiple of
 * 16 in [16, 512]; hq, hkv <= 4096; batch * seqlen < 2^32.  hq = 0 rotates k
 * only (q and its output are then not read and may be NULL): the pass that
 * goes with siq_attn_rope_fwd_plan / _bwd_plan, which rotate q themselves.
 * No workspace.
 * ------------------------------------------------------------------------- */
int siq_rope_fwd(const void* q, const void* k, const void* cos, const void* sin, void* q_embed, void* k_embed,
                 int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides, void* stream);

int siq_rope_bwd(const void* dq_embed, const void* dk_embed, const void* cos, const void* sin, void* dq, void* dk,
                 int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides, void* stream);

/* The same two passes with the dtype of cos / sin chosen (cs_dtype:
 * SIQ_DTYPE_BF16 = siq_rope_fwd / _bwd, or SIQ_DTYPE_FP32).  fp32 cos / sin
 * are what transformers' rotary embedding hands over under bf16 autocast
 * over fp32 master weights (the reference's bf16=True training,
 * scripts/train.py:712): there q and k are bf16 (autocast Linear outputs) and
 * torch promotes q * cos + rotate_half(q) * sin to fp32, which the attention
 * then casts to bf16.  siq_rope_fwd_ex writes that bf16 cast directly:
 * q_embed = rb(fl(fl(q1 c1) - fl(q2 s1)), ...) with fp32 products and sum and
 * one rounding to bf16, bitwise the reference's q_embed.to(bf16).
 * siq_rope_bwd_ex is the reference's autograd of those ops on the bf16
 * gradient of that cast: dq = rb(rb(fl(g1 c1)) + rb(fl(g2 s2))), ... .  With
 * fp32 cos / sin their strides are multiples of 4 elements (16 bytes); the
 * other tensors are as for siq_rope_fwd. */
int siq_rope_fwd_ex(const void* q, const void* k, const void* cos, const void* sin, void* q_embed, void* k_embed,
                    int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides,
                    int cs_dtype, void* stream);

int siq_rope_bwd_ex(const void* dq_embed, const void* dk_embed, const void* cos, const void* sin, void* dq, void* dk,
                    int64_t batch, int64_t seqlen, int hq, int hkv, int head_dim, const int64_t* strides,
                    int cs_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Pixel-shuffle projector (the vision-to-text bridge).
 *
 * Replaces SiQ_VLProjector.forward (siq_vl/model/modeling.py:100-105): the
 * pixel shuffle of :74-98 (view [batch, side, side, dv], reshape by the
 * factor r, permute(0, 1, 3, 2, 4, 5), reshape to [batch, (side/r)^2,
 * r*r*dv]) followed by the bias-free Linear mlp (:59) -- and its autograd
 * backward -- without materialising the shuffled tensor:
 *   y [batch*(side/r)^2, out_features] = shuffle(x) weight^T,
 *   dx = unshuffle(dy weight),  dweight = dy^T shuffle(x).
 * x [batch, side*side, vision_dim], weight [out_features, r*r*vision_dim],
 * y / dy [batch*(side/r)^2, out_features]: bf16, contiguous, 16-byte
 * aligned; fp32 accumulation.  vision_dim % 64 == 0, out_features % 8 == 0,
 * side % r == 0; x, y and weight each < 2^31 elements, tokens < 2^24.
 * siq_proj_bwd: dx and/or dweight may be NULL (not computed).  Workspace:
 * siq_proj_workspace_bytes (split-K partial sums; may be 0).  Deterministic.
 * ------------------------------------------------------------------------- */
size_t siq_proj_workspace_bytes(int64_t batch, int64_t side, int64_t vision_dim, int factor, int64_t out_features);

int siq_proj_fwd(const void* x, const void* weight, void* y, int64_t batch, int64_t side, int64_t vision_dim,
                 int factor, int64_t out_features, void* workspace, size_t workspace_bytes, void* stream);

int siq_proj_bwd(const void* x, const void* weight, const void* dy, void* dx, void* dweight, int64_t batch,
                 int64_t side, int64_t vision_dim, int factor, int64_t out_features, void* workspace,
                 size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Vision-token splice fused with the embedding gather.
 *
 * Replaces, in SiQ_VLForCausalLM.forward (siq_vl/model/modeling.py:252-270),
 * the embedding lookup of input_ids (:253), the nonzero() of the image-token
 * positions (:257), their count check (:259-267) and the index assignment of
 * the flattened vision rows (:269-270):
 *   out[p] = vision[r]          if input_ids[p] == image_token_id, r = number
 *                               of image tokens before p (row-major order);
 *   out[p] = weight[input_ids[p]] otherwise.
 * input_ids [n_tokens] int64; weight [vocab, hidden], vision [n_vision,
 * hidden], out [n_tokens, hidden]: bf16, contiguous, 16-byte aligned;
 * hidden % 8 == 0.  Outputs (device): image_pos [n_vision] int32 = token index
 * of vision row r; counts[0] = image tokens found (the caller raises the
 * reference's ValueError when it differs from n_vision: rows of image tokens
 * beyond n_vision are written as zeros), counts[1] = ids outside [0, vocab)
 * (written as zeros; the reference's embedding would raise).  Workspace:
 * siq_splice_workspace_bytes(n_tokens).
 *
 * siq_gather_rows: dst[i] = src[rows[i]], i < n (rows of hidden bf16): the
 * backward's vision-row gradient (IndexPutBackward of :270) from image_pos;
 * rows[i] < 0 gives a zero row (image_pos slots past the image tokens found
 * hold -1).  The splice and the gather only copy 16-byte chunks of rows, so
 * rows of another dtype are passed as their bf16 view (an fp32 row of H
 * elements as 2H bf16).
 * ------------------------------------------------------------------------- */
size_t siq_splice_workspace_bytes(int64_t n_tokens);

int siq_splice_fwd(const int64_t* input_ids, int64_t n_tokens, const void* weight, int64_t vocab, int64_t hidden,
                   const void* vision, int64_t n_vision, int64_t image_token_id, void* out, int32_t* image_pos,
                   int64_t* counts, void* workspace, size_t workspace_bytes, void* stream);

int siq_gather_rows(const void* src, const int32_t* rows, int64_t n, int64_t hidden, void* dst, void* stream);

/* ---------------------------------------------------------------------------
 * Embedding-table gradient of the splice (the text model's input embeddings).
 *
 * Replaces the backward of the embedding lookup at siq_vl/model/modeling.py:253
 * together with the index assignment at :270 (IndexPutBackward zeroes the
 * overwritten image rows before the embedding backward): torch's
 * embedding_dense_backward with the image token as padding index.
 *   dweight[v] = sum of grad[p] over tokens p with input_ids[p] == v,
 * for v in [0, vocab) other than skip_id0 / skip_id1 (the image token and the
 * table's padding index; -1 for none); every other row is zero.  The sum is
 * fp32, in the order of torch's sorted embedding backward (each id's tokens
 * in position order, partial sums of at most 10 rows added in order), rounded
 * once; deterministic.  grad [n_tokens, hidden] and dweight [vocab, hidden]
 * contiguous, 16-byte aligned, both bf16 (dtype SIQ_DTYPE_BF16) or both fp32
 * (SIQ_DTYPE_FP32, the reference's fp32 master weights); hidden % 8 == 0.
 * Workspace: siq_embedding_bwd_workspace_bytes(n_tokens, vocab).
 * ------------------------------------------------------------------------- */
size_t siq_embedding_bwd_workspace_bytes(int64_t n_tokens, int64_t vocab);

int siq_embedding_bwd(const void* grad, const int64_t* input_ids, int64_t n_tokens, int64_t vocab, int64_t hidden,
                      int dtype, int64_t skip_id0, int64_t skip_id1, void* dweight, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Measurement support (no reference counterpart).
 *
 * siq_probe_clock: one wave per CU spins for about spin_ticks ticks of the
 * constant 100 MHz counter and writes out[0] = shader-clock cycles elapsed,
 * out[1] = 100 MHz ticks elapsed (device uint64[2]); the shader clock the GPU
 * ran at is out[0] / out[1] * 100 MHz.  spin_ticks in [1, 1e8].
 * ------------------------------------------------------------------------- */
int siq_probe_clock(uint64_t* out, int64_t spin_ticks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SIQ_KERNELS_H */
