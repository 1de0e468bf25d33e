/*
 * fa_mi355x.h -- C ABI of the MI355X (gfx950) FlashAttention library.
 *
 * Plain C: raw device pointers, element strides, sizes, an opaque stream
 * handle (a hipStream_t passed as void*; NULL means the default stream).
 * No torch, HIP or C++ types cross this boundary, nothing throws, and the
 * library never allocates or frees device memory: the caller passes every
 * output and the backward workspace.
 *
 * Tensor convention (same as the Python API this library backs):
 *   q, k, v, o, do, dq, dk, dv : (B, S, H, D) fp16 (IEEE binary16; bf16 too
 *                                 in fa_fwd_gqa / fa_bwd_gqa), any
 *                                 strides with the D stride equal to 1;
 *   lse, delta                 : (B, H, S) fp32, contiguous.
 * Strides are in elements and given per tensor as {b, s, h, d}.
 * All launches are asynchronous on `stream`; no call synchronises the host.
 * Kernels run on the device `stream` belongs to (the current device for
 * the NULL stream), whichever device is current in the calling thread, and
 * every pointer must be memory of that device; launch decisions (the
 * device's CU count) and fa_bwd_gqa_noalloc's scratch buffer follow that
 * device too.
 *
 * Status codes: 0 on success, a negative FA_ERR_* otherwise. Argument
 * validation runs before any HIP call, so it behaves the same on a machine
 * without a GPU.
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 9

/* Size of the static device scratch buffer that fa_bwd_gqa_noalloc uses as
 * its workspace (one per GPU, held for the life of the process). */
#define FA_NOALLOC_SCRATCH_BYTES (64u << 20)

enum fa_status {
  FA_OK = 0,
  FA_ERR_NULL_POINTER = -1,   /* a required pointer is NULL                 */
  FA_ERR_HEAD_DIM = -2,       /* D not in {32, 64, 128}                     */
  FA_ERR_SHAPE = -3,          /* B, a sequence length or a head count <= 0,
                                 or H not a multiple of Hk                  */
  FA_ERR_STRIDE = -4,         /* D stride != 1, a stride not a multiple of
                                 8 elements (16-byte vector access), or an
                                 output whose (b, s, h) rows overlap        */
  FA_ERR_ALIGNMENT = -5,      /* a base pointer not 16-byte aligned         */
  FA_ERR_SCALE = -6,          /* sm_scale not finite                        */
  FA_ERR_WORKSPACE = -7,      /* workspace NULL or smaller than required    */
  FA_ERR_TOO_LARGE = -8,      /* sizes whose element offsets overflow int64,
                                 a sequence stride over ~8.45e6 elements
                                 (127 rows of a 128-row tile must span
                                 < 2^31 bytes: 32-bit offsets), or
                                 a grid beyond the launch limits            */
  FA_ERR_LAUNCH = -9,         /* the HIP runtime rejected a kernel launch
                                 (or a device query it needed)              */
  FA_ERR_DTYPE = -10,         /* dtype not one of enum fa_dtype             */
  FA_ERR_EPS = -11,           /* norm eps negative or not finite            */
  FA_ERR_SCRATCH = -12        /* fa_bwd_gqa_noalloc: the problem's delta does
                                 not fit FA_NOALLOC_SCRATCH_BYTES           */
};

/* Element type of the 16-bit tensors (fa_fwd_gqa / fa_bwd_gqa; the other
 * entry points are fp16, like the reference). */
enum fa_dtype {
  FA_DTYPE_F16 = 0,           /* IEEE binary16                              */
  FA_DTYPE_BF16 = 1           /* bfloat16                                   */
};

/* Version of this ABI (FA_ABI_VERSION of the build). */
int fa_abi_version(void);

/* Static, NUL-terminated description of a status code. Never NULL. */
const char *fa_strerror(int status);

/*
 * Forward attention: o = softmax(sm_scale * q k^T [+ causal mask]) v.
 * When `lse` is non-NULL it receives the natural-log log-sum-exp of each
 * score row, (B, H, S) fp32 contiguous; +inf marks a row with no visible key.
 *
 * Replaces flash_attn_volta/triton_fa.py:291-397 (flash_attn_forward and
 * _run_kernel, launching _fa_fwd_kernel_d64 / _fa_fwd_kernel_d128 at
 * triton_fa.py:381-392). Unlike that wrapper it reads the (B,S,H,D)
 * strides directly, so no permute copies and no zero padding of D=32.
 */
int fa_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
           int B, int S, int H, int D,
           const int64_t q_strides[4], const int64_t k_strides[4],
           const int64_t v_strides[4], const int64_t o_strides[4],
           float sm_scale, int causal, void *stream);

/*
 * Grouped-query / multi-query attention with separate query and key
 * lengths: q, o are (B, Sq, H, D); k, v are (B, Sk, Hk, D) with H a
 * multiple of Hk, and query head h attends with key/value head
 * h / (H / Hk) (the head order of HuggingFace's repeat_kv); lse is
 * (B, H, Sq).  `causal` aligns the mask to the bottom right: query i sees
 * key j iff j <= i + (Sk - Sq), so the last query sees every key (the
 * KV-cache / chunked-prefill convention); a query that sees no key gets
 * o = 0 and lse = +inf.  `dtype` (enum fa_dtype) is the element type of
 * q, k, v and o; accumulation is fp32 either way.  With Sq == Sk, Hk == H
 * and FA_DTYPE_F16 it is fa_fwd.
 *
 * No counterpart in the reference kernels, whose wrapper asserts equal
 * q/k/v shapes (flash_attn_volta/triton_fa.py:315); it replaces the
 * repeat_kv expansion of K/V the reference's HuggingFace patch does before
 * calling them (flash_attn_volta/patch_hf.py:186-188, 470-471) and that
 * patch's fallback to the original attention when a KV cache makes
 * q_len != kv_len (patch_hf.py:145-162).
 */
int fa_fwd_gqa(const void *q, const void *k, const void *v, void *o, float *lse,
               int B, int Sq, int Sk, int H, int Hk, int D,
               const int64_t q_strides[4], const int64_t k_strides[4],
               const int64_t v_strides[4], const int64_t o_strides[4],
               float sm_scale, int causal, int dtype, void *stream);

/*
 * fa_fwd_gqa for a short block of queries against a long key sequence
 * (decode and speculative-decode steps with a KV cache), given a
 * workspace: when every key/value head's group of query rows fits one
 * 64-row tile (H / Hk * Sq <= 64), the regular grid would leave the GPU
 * under-filled and Sk >= 256, the keys are split into ranges processed by
 * separate workgroups, each key/value head's query heads share every K/V
 * tile, and a second kernel merges the ranges through their log-sum-exps;
 * otherwise it is exactly fa_fwd_gqa (the workspace is not touched).
 * Same arguments and results as fa_fwd_gqa (to fp32 rounding of the merge).
 *
 * No counterpart in the reference, whose HF patch falls back to eager
 * attention whenever a KV cache has content (flash_attn_volta/patch_hf.py:
 * 145-162).
 */
int fa_fwd_splitkv(const void *q, const void *k, const void *v, void *o, float *lse,
                   void *workspace, size_t workspace_bytes,
                   int B, int Sq, int Sk, int H, int Hk, int D,
                   const int64_t q_strides[4], const int64_t k_strides[4],
                   const int64_t v_strides[4], const int64_t o_strides[4],
                   float sm_scale, int causal, int dtype, void *stream);

/* Workspace bytes fa_fwd_splitkv needs for these sizes on the current
 * device (its compute-unit count sets the split), 0 when it would not split
 * (or for invalid sizes). */
size_t fa_fwd_splitkv_workspace_bytes(int B, int Sq, int Sk, int H, int Hk, int D);

/*
 * Forward with a workspace: the schedule that is fastest for these sizes.
 * Same arguments and results as fa_fwd_gqa (to fp32 rounding of a merge),
 * plus `workspace`, `workspace_bytes`.
 *   - Short query blocks against long keys: fa_fwd_splitkv's key split.
 *   - Causal, Sq == Sk, at least 32 query tiles of 64 rows per head and at
 *     most half a tile per compute unit in the plain grid (one from 48
 *     tiles per head, 1.75 from 64): query tiles paired
 *     light with heavy (tile p with tile nb - 1 - p), each pair cut in
 *     three work items of about a third of the pair each (the heavy tile's
 *     two key halves, the light tile); the heavy tile's halves go to the
 *     workspace in fp32 and a second kernel merges them through their
 *     log-sum-exps.  The plain schedule ends on the heaviest query tiles,
 *     each sweeping every key tile alone on its compute unit.
 *   - Otherwise: fa_fwd_gqa, the workspace untouched.
 * A workspace smaller than fa_fwd_workspace_bytes (NULL / 0 included)
 * selects the plain forward; a used workspace must be 16-byte aligned.
 *
 * No counterpart in the reference, whose causal kernel sweeps each query
 * block's keys in one program (flash_attn_volta/triton_fa.py:110-117).
 */
int fa_fwd_ws(const void *q, const void *k, const void *v, void *o, float *lse,
              void *workspace, size_t workspace_bytes,
              int B, int Sq, int Sk, int H, int Hk, int D,
              const int64_t q_strides[4], const int64_t k_strides[4],
              const int64_t v_strides[4], const int64_t o_strides[4],
              float sm_scale, int causal, int dtype, void *stream);

/* Workspace bytes with which fa_fwd_ws runs its fastest schedule for these
 * sizes on the current device (its compute-unit count decides), 0 when the
 * plain forward is that schedule (or for invalid sizes). */
size_t fa_fwd_workspace_bytes(int B, int Sq, int Sk, int H, int Hk, int D, int causal);

/*
 * Backward pre-pass: delta[b,h,s] = sum_d o[b,s,h,d] * do[b,s,h,d] in fp32.
 * Replaces the torch expression at flash_attn_volta/triton_fa_bwd.py:649-650.
 *
 * With `rowmax` non-NULL it also writes the row-group maxima the dK/dV
 * kernel reads (fa_bwd_dkdv, fa_bwd_blocks): for every group of 32 query
 * rows of each (b, h), rowmax[b][h][g][0] = max over the group's rows and
 * d of |do[b, s, h, d]| and rowmax[b][h][g][1] = max |delta[b, h, s]|,
 * fp32, g < ceil(S / 32), fa_bwd_rowmax_bytes(B, S, H) bytes, 16-byte
 * aligned.  (No reference counterpart: they bound |dS| so that the dK/dV
 * kernel fixes its fp16 dS scale per query tile; see fa_bwd.)
 */
int fa_bwd_preprocess(const void *o, const void *dout, float *delta, float *rowmax,
                      int B, int S, int H, int D,
                      const int64_t o_strides[4], const int64_t do_strides[4],
                      void *stream);

/* Bytes of the row-group maxima of fa_bwd_preprocess (0 on bad sizes). */
size_t fa_bwd_rowmax_bytes(int B, int S, int H);

/* Bytes of device workspace fa_bwd needs for these sizes (0 on bad sizes):
 * delta and the row-group maxima. */
size_t fa_bwd_workspace_bytes(int B, int S, int H, int D);

/*
 * Bytes of device workspace with which fa_bwd / fa_bwd_gqa run their
 * fastest schedule for these sizes (0 on bad sizes): the
 * fa_bwd_workspace_bytes minimum plus, for causal D = 64 / 128 problems
 * whose dQ grid is at most half a round of resident workgroups (and whose
 * last query block sweeps at least 64 key tiles, 48 at D = 128, where the fused launch
 * below could run instead), room for the query-block split of the dQ kernel (its longest query blocks swept
 * by two workgroups, fp32 halves added by the dK/dV kernel) and, when the
 * key blocks fit one round, for the key-block split beside it (the
 * longest causal key blocks swept by two workgroups each, fp32 partials
 * added by whichever finishes second): at most 80 MiB + 4 KiB more.
 * (Without the dQ split the causal backward runs its fused launch,
 * unsplit, which measured faster.)
 * Any workspace of at least the minimum is valid: with less than this
 * size the backward runs unsplit.  Split and unsplit results differ in
 * rounding only; each is bit-reproducible.
 *
 * No counterpart in the reference (its backward has no workspace,
 * flash_attn_volta/triton_fa_bwd.py:636-700).
 */
size_t fa_bwd_gqa_workspace_bytes(int B, int Sq, int Sk, int H, int Hk, int D, int causal);

/*
 * Backward attention: (dq, dk, dv) of L = <o, dout> with o = fa_fwd(q,k,v),
 * given the forward's `lse`. Two launches. Causal with D = 32 or 64, and
 * causal D = 128 on grids of at most four workgroups of eight waves per
 * compute unit, in both cases without the dQ query-block split (see
 * fa_bwd_gqa_workspace_bytes) and unsplit:
 * fa_bwd_preprocess's kernel (delta = rowsum(o * dout) and the row-group
 * maxima into the workspace), then one launch running every dK/dV
 * workgroup (one per key block, or two for the longest blocks when the
 * workspace has room: fa_bwd_gqa_workspace_bytes) and then every dQ
 * workgroup (one per query block). Otherwise: the dQ kernel, which also
 * computes delta and the maxima into the workspace, then the dK/dV kernel.
 * dS is rounded to fp16 for the MFMAs at a power-of-two scale per key,
 * settled per 32- to 128-query tile from the bound |dS| <= max|do| *
 * ||v_key||_1 + max|delta| over the tile's rows (so no scaled dS can
 * overflow fp16, and tiny upstream gradients keep fp16 precision), and
 * unscaled in fp32 at the end. No floating-point atomics: results
 * are bit-reproducible and, with the fa_bwd_workspace_bytes workspace (no
 * split), bit-identical to the three separate calls fa_bwd_preprocess,
 * fa_bwd_dq, fa_bwd_dkdv.
 *
 * Replaces flash_attn_volta/triton_fa_bwd.py:587-700 (flash_attn_backward
 * and _run_bwd_kernels, launching _fa_bwd_dq_kernel_* and
 * _fa_bwd_dkdv_kernel_* at triton_fa_bwd.py:667-695).
 */
int fa_bwd(const void *dout, const void *q, const void *k, const void *v,
           const void *o, const float *lse,
           void *dq, void *dk, void *dv,
           void *workspace, size_t workspace_bytes,
           int B, int S, int H, int D,
           const int64_t do_strides[4], const int64_t q_strides[4],
           const int64_t k_strides[4], const int64_t v_strides[4],
           const int64_t o_strides[4], const int64_t dq_strides[4],
           const int64_t dk_strides[4], const int64_t dv_strides[4],
           float sm_scale, int causal, void *stream);

/*
 * Backward of fa_fwd_gqa: dq is (B, Sq, H, D), dk and dv are (B, Sk, Hk, D)
 * and hold the sums over the H / Hk query heads that share each key/value
 * head (computed in the kernel, in a fixed order: still bit-reproducible).
 * The workspace is fa_bwd_workspace_bytes(B, Sq, H, D).  Same masking and
 * dtype convention as fa_fwd_gqa (every 16-bit tensor, inputs and
 * gradients, has element type `dtype`); with Sq == Sk, Hk == H and
 * FA_DTYPE_F16 it is fa_bwd.
 *
 * No counterpart in the reference kernels (see fa_fwd_gqa); it replaces
 * autograd through the reference patch's repeat_kv
 * (flash_attn_volta/patch_hf.py:186-188, 470-471).
 */
int fa_bwd_gqa(const void *dout, const void *q, const void *k, const void *v,
               const void *o, const float *lse,
               void *dq, void *dk, void *dv,
               void *workspace, size_t workspace_bytes,
               int B, int Sq, int Sk, int H, int Hk, int D,
               const int64_t do_strides[4], const int64_t q_strides[4],
               const int64_t k_strides[4], const int64_t v_strides[4],
               const int64_t o_strides[4], const int64_t dq_strides[4],
               const int64_t dk_strides[4], const int64_t dv_strides[4],
               float sm_scale, int causal, int dtype, void *stream);

/*
 * fa_bwd_gqa for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the same arguments minus the workspace, which is a static
 * device buffer of FA_NOALLOC_SCRATCH_BYTES that the library holds per GPU
 * for the life of the process.  delta (4 * B * H * Sq bytes) must fit it,
 * else FA_ERR_SCRATCH (checked before any HIP call); the split schedule of
 * fa_bwd_gqa_workspace_bytes runs when it fits too, and results are then
 * bit-identical to fa_bwd_gqa given a workspace of the same size.  Calls
 * and allocates nothing else: no hipMalloc, no memset.
 *
 * Every call on a GPU shares that GPU's buffer, so calls that overlap on
 * one GPU (concurrent streams, or host threads without ordering) race and
 * must be serialised by the caller.  The buffer used is that of the
 * stream's device; its address is looked up on the first call per device
 * (hipGetSymbolAddress, which allocates nothing), so a caller that
 * captures this call into a HIP graph makes one eager call on the device
 * first.
 *
 * No counterpart in the reference (its backward allocates through torch,
 * flash_attn_volta/triton_fa_bwd.py:650-654).
 */
int fa_bwd_gqa_noalloc(const void *dout, const void *q, const void *k, const void *v,
                       const void *o, const float *lse,
                       void *dq, void *dk, void *dv,
                       int B, int Sq, int Sk, int H, int Hk, int D,
                       const int64_t do_strides[4], const int64_t q_strides[4],
                       const int64_t k_strides[4], const int64_t v_strides[4],
                       const int64_t o_strides[4], const int64_t dq_strides[4],
                       const int64_t dk_strides[4], const int64_t dv_strides[4],
                       float sm_scale, int causal, int dtype, void *stream);

/*
 * The two main backward kernels as separate steps (outside its fused
 * causal launch, fa_bwd runs the dQ kernel, computing delta
 * and the maxima on the way, then the dK/dV kernel; called separately they
 * take both from fa_bwd_preprocess).  `delta` is the
 * fa_bwd_preprocess output, (B, H, S) fp32 contiguous, and fa_bwd_dkdv's
 * `rowmax` (not NULL) its row-group maxima for the same o and dout.
 *
 * fa_bwd_dkdv replaces the launch of _fa_bwd_dkdv_kernel_{d64,d128}
 * (flash_attn_volta/triton_fa_bwd.py:682-695): dK, dV per key block.
 * fa_bwd_dq replaces the launch of _fa_bwd_dq_kernel_{d64,d128}
 * (triton_fa_bwd.py:667-679): dQ per query block.
 */
int fa_bwd_dkdv(const void *dout, const void *q, const void *k, const void *v,
                const float *lse, const float *delta, const float *rowmax, void *dk, void *dv,
                int B, int S, int H, int D,
                const int64_t do_strides[4], const int64_t q_strides[4],
                const int64_t k_strides[4], const int64_t v_strides[4],
                const int64_t dk_strides[4], const int64_t dv_strides[4],
                float sm_scale, int causal, void *stream);

int fa_bwd_dq(const void *dout, const void *q, const void *k, const void *v,
              const float *lse, const float *delta, void *dq,
              int B, int S, int H, int D,
              const int64_t do_strides[4], const int64_t q_strides[4],
              const int64_t k_strides[4], const int64_t v_strides[4],
              const int64_t dq_strides[4],
              float sm_scale, int causal, void *stream);

/*
 * Both gradient launches of fa_bwd given delta and the row-group maxima
 * (the fa_bwd_preprocess outputs, `rowmax` not NULL), i.e. fa_bwd without
 * its delta step and without a workspace (so
 * without the key-block split): where fa_bwd takes its fused launch
 * (above), that launch of every dK/dV and every dQ workgroup, otherwise
 * fa_bwd_dq then fa_bwd_dkdv.  Bit-identical to fa_bwd with the fa_bwd_workspace_bytes
 * workspace.  For callers that time or schedule the gradient launches
 * apart from the delta step.
 *
 * Replaces the two kernel launches of _run_bwd_kernels, which take delta
 * from the torch op before them (flash_attn_volta/triton_fa_bwd.py:667-695).
 */
int fa_bwd_blocks(const void *dout, const void *q, const void *k, const void *v,
                  const float *lse, const float *delta, const float *rowmax, void *dq,
                  void *dk, void *dv, int B, int S, int H, int D,
                  const int64_t do_strides[4], const int64_t q_strides[4],
                  const int64_t k_strides[4], const int64_t v_strides[4],
                  const int64_t dq_strides[4], const int64_t dk_strides[4],
                  const int64_t dv_strides[4],
                  float sm_scale, int causal, void *stream);

/*
 * Fused attention prologue for q and k: optional per-head RMSNorm (QK-norm)
 * followed by rotary position embedding in the rotate-half form.  For each
 * row x (one (b, s, head) of D elements) of q and of k:
 *
 *   y = w * x / sqrt(mean(x^2) + eps)      when that side's norm weight w
 *   y = x                                  is given, else
 *   out[d]       = y[d] cos[d]         - y[d + D/2] sin[d]        (d < D/2)
 *   out[d + D/2] = y[d + D/2] cos[d + D/2] + y[d] sin[d + D/2]
 *
 * computed in fp32 and rounded once.  q, q_out: (B, S, H, D); k, k_out:
 * (B, S, Hk, D), strides {b, s, h, d} as for the attention calls; cos, sin:
 * (B or 1, S, D) tables of the same dtype with element strides
 * cs_strides = {b, s} (d stride 1; b stride 0 shares one table across the
 * batch); q_norm_weight / k_norm_weight: (D) of the same dtype, or NULL for
 * no norm on that side; eps is used only with a weight.  D in {16, 32, 64,
 * 128}; dtype is FA_DTYPE_F16 or FA_DTYPE_BF16.
 *
 * Replaces the prologue the reference leaves to transformers before its
 * attention call: Qwen3's q_norm / k_norm then apply_rotary_pos_emb
 * (flash_attn_volta/patch_hf.py:291-303), and apply_rotary_pos_emb alone
 * for Qwen2 / Llama (patch_hf.py:177, :462).  The reference lists the fused
 * QK-norm as not landed (PERF.md:99-104).
 */
int fa_rope_qk_fwd(const void *q, const void *k, void *q_out, void *k_out,
                   const void *cos, const void *sin,
                   const void *q_norm_weight, const void *k_norm_weight, float eps,
                   int B, int S, int H, int Hk, int D,
                   const int64_t q_strides[4], const int64_t k_strides[4],
                   const int64_t q_out_strides[4], const int64_t k_out_strides[4],
                   const int64_t cs_strides[2], int dtype, void *stream);

/* Bytes of workspace fa_rope_qk_bwd needs when a norm weight is given (0 for
 * an invalid shape).  Depends only on the sizes. */
size_t fa_rope_qk_workspace_bytes(int B, int S, int H, int Hk, int D);

/*
 * Backward of fa_rope_qk_fwd: from the gradients of q_out / k_out, the
 * gradients of q / k, and for a normed side the gradient of its weight,
 * (D) fp32, reduced in a fixed order (reproducible).  q / k (the forward's
 * inputs), dq_norm_weight / dk_norm_weight and the workspace are read only
 * for a side with a norm weight and may be NULL otherwise.
 */
int fa_rope_qk_bwd(const void *dq_out, const void *dk_out, const void *q, const void *k,
                   const void *cos, const void *sin,
                   const void *q_norm_weight, const void *k_norm_weight, float eps,
                   void *dq, void *dk, float *dq_norm_weight, float *dk_norm_weight,
                   void *workspace, size_t workspace_bytes,
                   int B, int S, int H, int Hk, int D,
                   const int64_t dq_out_strides[4], const int64_t dk_out_strides[4],
                   const int64_t q_strides[4], const int64_t k_strides[4],
                   const int64_t dq_strides[4], const int64_t dk_strides[4],
                   const int64_t cs_strides[2], int dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_MI355X_H */
