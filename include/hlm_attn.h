/*
 * hlm_attn.h -- C ABI of the MI355X (gfx950) causal sliding-window attention
 * library libhlm_attn.so.
 *
 * This is the device boundary that hackable-lm's attention backends cross:
 * the reference calls `flash_attn_func(q, k, v, dropout_p, causal=True,
 * window_size=(W - 1, 0))` from `kernels.scaled_dot_product_attention`
 * (/root/reference/kernels.py:836-841), reached from
 * `AttentionCore.fwd_flash_attn_2` (/root/reference/model.py:216-226), and
 * autograd then runs FlashAttention-2's backward.  The two entry points below
 * replace that forward and that backward.
 *
 * Tensor conventions (all device pointers, caller-owned):
 *   q, o, dO, dq          bf16 (B, T, H,   D)
 *   k, v, dk, dv          bf16 (B, T, Hkv, D)
 *   lse                   fp32 (B, H, T), contiguous
 *   delta_ws              fp32 workspace of 2 * B * H * T floats
 * Each bf16 tensor has unit stride along D; its batch/time/head strides are
 * given in ELEMENTS as int64_t[3] = {stride_b, stride_t, stride_h}.  Every
 * stride must be a multiple of 8 and every bf16 base pointer 16-byte aligned
 * (so rows can be moved with 128-bit accesses), stride_t >= D (rows do not
 * overlap), and (T + 512) * stride_t * 2 must stay below 2^31 (rows are
 * addressed with 32-bit byte offsets); v may be a strided view of a fused
 * qkv projection (model.py:92-99).
 *
 * Mask: query i attends to keys j with  i - window < j <= i.
 *   window <= 0 or window >= T  ->  plain causal (the reference's `None`
 *   window, model.py:155-159).  This is FlashAttention's (window - 1, 0).
 * Supported: D in {64, 128}; H % Hkv == 0 (Hkv < H is grouped-query
 * attention); scale > 0 (the reference uses 1/sqrt(D)).
 *
 * Semantics: no allocation, no host synchronisation; all work is enqueued on
 * `stream` (a hipStream_t), so calls are safe inside HIP graph capture.
 * Return value: 0 on success, a negative HLM_ATTN_E* code otherwise; the
 * message is available from hlm_attn_last_error() on the calling thread.
 */
#ifndef HLM_ATTN_H
#define HLM_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HLM_ATTN_OK 0
#define HLM_ATTN_EINVAL (-1)      /* bad pointer, shape, stride or alignment */
#define HLM_ATTN_EUNSUPPORTED (-2) /* valid request this library does not implement */
#define HLM_ATTN_ELAUNCH (-3)     /* the HIP runtime rejected a kernel launch */

/* Largest nsplit hlm_attn_fwd_split accepts. */
#define HLM_ATTN_MAX_SPLIT 16

/* Element types of the rotary tables (cos, sin) of hlm_qk_norm_rope_*. */
#define HLM_TABLE_F32 0
#define HLM_TABLE_BF16 1

/* Element types of hlm_ce_rows' logits (the same codes). */
#define HLM_DTYPE_F32 0
#define HLM_DTYPE_BF16 1

/* ABI revision of this header; bumped on any signature change. */
int hlm_attn_abi_version(void);

/*
 * Forward: o = softmax(scale * q k^T + mask) v, lse = logsumexp of the same
 * masked scores (natural log, fp32).
 * Replaces flash_attn_func(q, k, v, dropout_p=0.0, causal=True,
 * window_size=(window - 1, 0)) at /root/reference/kernels.py:841 and the
 * `torch` math at /root/reference/kernels.py:785-800.
 */
int hlm_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                 int B, int T, int H, int Hkv, int D,
                 const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides,
                 int window, float scale, void* stream);

/*
 * Split-key forward for small grids (the evaluation harness's calls at batch
 * 1 and ragged T, lm_eval_hackable_lm.py:134-160,185-207, where B * H * T/128
 * query tiles leave most of the chip idle and the longest row's key tiles set
 * the time).  Same inputs, outputs and semantics as hlm_attn_fwd; nsplit
 * workgroups share each query tile's key range and a second kernel merges
 * their partial results by their log-sum-exp.  ws is caller-allocated device
 * memory of nsplit * B * H * T * (D + 2) floats, 16-byte aligned (fully
 * overwritten; no initialisation needed); nsplit in [1, HLM_ATTN_MAX_SPLIT]
 * (1 is hlm_attn_fwd, and ws may then be null).  Results agree with
 * hlm_attn_fwd within bf16 rounding of O (the partial sums are fp32).  No
 * counterpart in the reference: FlashAttention-2's forward is one call.
 */
int hlm_attn_fwd_split(const void* q, const void* k, const void* v, void* o, float* lse, float* ws, int nsplit,
                       int B, int T, int H, int Hkv, int D, const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* o_strides, int window, float scale,
                       void* stream);

/*
 * The nsplit this library recommends for hlm_attn_fwd_split on an MI355X:
 * 1 (use hlm_attn_fwd) unless the query tiles fill less than half of the
 * chip's workgroup slots and the longest row spans at least 24 key tiles of
 * 64 (shorter rows run faster unsplit than split and merged); then one split
 * per 12 key tiles of the longest row.  Pure function of the shape; touches
 * no device.
 */
int hlm_attn_fwd_split_count(int B, int T, int H, int D, int window);

/*
 * Backward: given dO and the forward's o and lse, writes dq, dk, dv (in the
 * layouts given by their strides).  delta_ws is a caller-provided fp32
 * workspace of 2 * B * H * T floats: it receives -lse * log2(e), then
 * -rowsum(dO * o), each as (B, H, T).  dk/dv are written completely (not
 * accumulated into).
 * Replaces the backward of flash_attn_func (FlashAttention-2's autograd
 * Function, called from /root/reference/kernels.py:841), i.e. the gradient
 * of the math at /root/reference/kernels.py:785-800.
 */
int hlm_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                 const float* lse, void* dq, void* dk, void* dv, float* delta_ws,
                 int B, int T, int H, int Hkv, int D,
                 const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                 const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
                 const int64_t* dk_strides, const int64_t* dv_strides,
                 int window, float scale, void* stream);

/*
 * The two phases of hlm_attn_bwd, same arguments, run in this order on one
 * stream: hlm_attn_bwd_dq writes dq and delta_ws; hlm_attn_bwd_dkdv reads
 * delta_ws and writes dk, dv.  hlm_attn_bwd == dq phase then dkdv phase.
 * Exposed so a caller can time or schedule the phases separately; the
 * reference has no counterpart (FlashAttention-2's backward is one call).
 */
int hlm_attn_bwd_dq(const void* q, const void* k, const void* v, const void* o, const void* dout,
                    const float* lse, void* dq, void* dk, void* dv, float* delta_ws,
                    int B, int T, int H, int Hkv, int D,
                    const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                    const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
                    const int64_t* dk_strides, const int64_t* dv_strides,
                    int window, float scale, void* stream);
int hlm_attn_bwd_dkdv(const void* q, const void* k, const void* v, const void* o, const void* dout,
                      const float* lse, void* dq, void* dk, void* dv, float* delta_ws,
                      int B, int T, int H, int Hkv, int D,
                      const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                      const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
                      const int64_t* dk_strides, const int64_t* dv_strides,
                      int window, float scale, void* stream);

/*
 * Single-pass backward (head_dim 64 only): the same gradients as
 * hlm_attn_bwd, with S and dP formed once per score block.  Three kernels
 * on `stream`: the delta workspace rows; one key-stationary pass that
 * writes dk, dv and per-key-tile dQ partials (bf16) into partial_ws; and a
 * reduce of the partials into dq.  dk and dv are bit-identical to
 * hlm_attn_bwd's; dq differs by the rounding of the partials.  partial_ws
 * (16-byte aligned) must hold hlm_attn_bwd_fused_workspace_bytes(B, T, H, D,
 * window) bytes, passed as partial_ws_bytes; other arguments as for
 * hlm_attn_bwd.  D != 64 returns HLM_ATTN_EUNSUPPORTED.  Replaces the same
 * call as hlm_attn_bwd (FlashAttention-2's backward behind
 * /root/reference/kernels.py:841); an alternative implementation of it,
 * selected by the caller.
 */
int hlm_attn_bwd_fused(const void* q, const void* k, const void* v, const void* o, const void* dout,
                       const float* lse, void* dq, void* dk, void* dv, float* delta_ws,
                       void* partial_ws, int64_t partial_ws_bytes,
                       int B, int T, int H, int Hkv, int D,
                       const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                       const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
                       const int64_t* dk_strides, const int64_t* dv_strides,
                       int window, float scale, void* stream);
/* Bytes of hlm_attn_bwd_fused's partial workspace: R * B * H * T * D * 2 with
 * R the most 128-key tiles one 32-row query tile meets (ceil((W - 1) / 128)
 * + 1 or fewer; ceil(T / 128) for plain causal).  Negative: an HLM_ATTN_E*
 * code (D != 64, bad shape). */
int64_t hlm_attn_bwd_fused_workspace_bytes(int B, int T, int H, int D, int window);

/*
 * hlm_attn_bwd without the caller's workspace: the same computation and
 * results as hlm_attn_bwd (bit for bit), with the workspace held in a
 * fixed device array inside the library, so the call allocates nothing
 * and needs no caller memory beyond inputs and outputs.  No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).
 * Limit: B * H * T <= 4,194,304 query rows (the array is 32 MiB per
 * device, held from the library's load until the process ends); larger
 * problems return HLM_ATTN_EUNSUPPORTED.  The first call on a device looks
 * up the array's device address once.  Calls on one device share the
 * array: calls that overlap in time on one device (on different streams)
 * race and must not be issued; calls on one stream are ordered and safe.
 */
int hlm_attn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o, const void* dout,
                         const float* lse, void* dq, void* dk, void* dv,
                         int B, int T, int H, int Hkv, int D,
                         const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                         const int64_t* o_strides, const int64_t* do_strides, const int64_t* dq_strides,
                         const int64_t* dk_strides, const int64_t* dv_strides,
                         int window, float scale, void* stream);

/*
 * The producer step before attention: fused RMSNorm (no weight) and partial
 * rotary embedding of q and k, forward and backward.  Per (batch, time, head)
 * row x of D values, in fp32:
 *   z = x * rsqrt(mean(x^2) + eps),
 *   out[d] = z[d] c - z[d+h] s (d < h), z[d] c + z[d-h] s (h <= d < R), z[d] (d >= R),
 * with R = rotary_dim, h = R / 2, c = cos[t * R + d mod h], s = sin[...].
 * q (B, T, H, D) and k (B, T, Hkv, D) are bf16 with unit D stride and
 * {stride_b, stride_t, stride_h} element strides (multiples of 8, 16-byte
 * aligned bases; stride_t >= D); cos and sin are (T, R) contiguous, 16-byte
 * aligned, of element type table_dtype (HLM_TABLE_F32 or HLM_TABLE_BF16: the
 * model's tables are bf16, model.py:62-70, and are read as they are);
 * q_out / k_out are bf16 and contiguous.  D in {64, 128}; R a multiple of 16
 * with 0 <= R <= D; B * T * (H + Hkv) < 2^31 - 1024; eps > 0.
 * Replaces kernels.qk_norm_rope_triton / the hackable_lm::qk_norm_rope Triton
 * op (/root/reference/kernels.py:441-535, :756-771), the math of
 * QKVProjection.fwd_torch (/root/reference/model.py:101-115).
 */
int hlm_qk_norm_rope_fwd(const void* q, const void* k, const void* cos, const void* sin, int table_dtype,
                         void* q_out, void* k_out, int B, int T, int H, int Hkv, int D, int rotary_dim,
                         const int64_t* q_strides, const int64_t* k_strides, float eps, void* stream);

/*
 * Its backward: given q, k (the forward's inputs) and grad_q_out, grad_k_out
 * (bf16, contiguous, the gradients of q_out / k_out), writes grad_q, grad_k
 * (bf16, contiguous):  gn = the rotation transposed applied to grad_out,
 * grad_x = r (gn - z mean(gn z)), r = rsqrt(mean(x^2) + eps).
 * Replaces the hackable_lm::qk_norm_rope_backward Triton op
 * (/root/reference/kernels.py:541-665) and its CPU closed form
 * (/root/reference/kernels.py:703-741).
 */
int hlm_qk_norm_rope_bwd(const void* q, const void* k, const void* grad_q_out, const void* grad_k_out,
                         const void* cos, const void* sin, int table_dtype, void* grad_q, void* grad_k,
                         int B, int T, int H, int Hkv, int D, int rotary_dim,
                         const int64_t* q_strides, const int64_t* k_strides, float eps, void* stream);

/*
 * The cross-entropy rows of the LM head's fused linear + cross-entropy, in
 * place: for each of n_rows rows of n_cols logits (bf16 or fp32 per
 * logits_dtype, rows row_stride elements apart) and its int64 target t,
 *   loss[row] = (logsumexp(x) - x_t) / n_tokens            (fp32)
 *   x_j      <- (softmax(x)_j - [j == t]) / n_tokens        (the gradient of
 *                                                           the mean loss)
 * computed in fp32.  A target equal to ignore_index gives a zero loss and a
 * zero gradient row (F.cross_entropy's rule); any other target outside
 * [0, n_cols) gives NaN for that row.  16-byte aligned rows (logits, n_cols
 * and row_stride multiples of 16 bytes) take a path that reads and writes
 * each row once.  Replaces the hackable_lm::linear_ce Triton op and its
 * kernel (/root/reference/kernels.py:286-336) inside the chunked fused
 * linear cross-entropy (/root/reference/kernels.py:878-959).
 */
int hlm_ce_rows(void* logits, int logits_dtype, int64_t row_stride, const int64_t* targets, float* loss, int n_rows,
                int n_cols, int64_t n_tokens, int ignore_index, void* stream);

/*
 * Residual add + RMSNorm (no weight) after an output or down projection:
 * for rows of n bf16 values (contiguous, 16-byte aligned, n a multiple of 8,
 * n <= 8192)
 *   out    = residual + branch                  (bf16, as the bf16 add rounds it)
 *   normed = out * rsqrt(mean(out^2) + eps)     (fp32 from the rounded out, bf16)
 * Replaces residual_rms_norm (/root/reference/model.py:73-75) in
 * OutputProjection.fwd_torch (/root/reference/model.py:261-264) and
 * DownProjection.fwd_torch (/root/reference/model.py:303-304).
 */
int hlm_residual_rms_norm_fwd(const void* residual, const void* branch, void* out, void* normed, int64_t rows, int n,
                              float eps, void* stream);

/*
 * Its backward: grad_in = grad_out + r (grad_normed - z mean(grad_normed z)),
 * r = rsqrt(mean(out^2) + eps), z = out r, from the forward's `out`; grad_in
 * is the gradient of both residual and branch.  Same layout rules.  (The
 * reference leaves this to autograd.)
 */
int hlm_residual_rms_norm_bwd(const void* out, const void* grad_out, const void* grad_normed, void* grad_in,
                              int64_t rows, int n, float eps, void* stream);

/* Message describing the last failed call on this thread ("" if none). */
const char* hlm_attn_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* HLM_ATTN_H */
