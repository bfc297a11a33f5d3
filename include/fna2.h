/*
 * fna2.h — C ABI of the MI355X (gfx950) FlashNaylisAttention-2 kernels.
 *
 * Attention score, per sequence and query head h (KV head h / (H / H_KV)):
 *
 *     S[i][j] = softmax_scale * <Q_i, K_j> + [h < H_G] * graph_scale[h] * <Rq_i, Rk_j>
 *
 * masked to -inf where j > i (causal, top-left aligned local positions) or
 * j >= len_k.  O_i = sum_j exp(S_ij - m_i) V_j / (l_i + 1e-6) and
 * LSE_i = m_i + log(l_i + 1e-6), as in the reference kernels
 * (myAiByMe/FNA2 FNA2/flash_naylis_attn.py:192-195, :340-345).
 *
 * Every entry point takes plain device pointers, element strides and sizes.
 * The library never allocates device memory: the caller owns every output
 * and the workspace (size it with fna2_*_workspace_bytes); the one exception
 * is fna2_fwd_noalloc's static 1 MiB array per GPU.  Kernels are
 * launched on the stream given; no call synchronises the host.  All entry
 * points are reentrant; the only state is a mutex-guarded record of the
 * last 256 plans forwards filled (see fna2_bwd_args.plan).  A nonzero return
 * means nothing was launched (FNA2_E_LAUNCH: a launch failed after earlier
 * launches of the same call may already have run).
 *
 * Layout.  Each tensor X is described by a base pointer and three element
 * strides (stride_b, stride_s, stride_h); the innermost (feature) stride
 * must be 1.  Dense mode (varlen == 0): element [b, h, s, f] lives at
 * X + b*stride_b + s*stride_s + h*stride_h + f.  Varlen mode: element
 * [t, h, f] of packed token t lives at X + t*stride_s + h*stride_h + f and
 * sequence b covers tokens [cu_seqlens[b], cu_seqlens[b+1]); stride_b is
 * ignored.  LSE and delta (fp32) use the same scheme with a feature size of 1.
 */
#ifndef FNA2_H_
#define FNA2_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FNA2_ABI_VERSION 3

/* Element types.  The attention entry points (fna2_fwd, fna2_bwd,
 * fna2_fwd_noalloc) take FNA2_BF16 or FNA2_F16 for q, k, v, out, dout, dq,
 * dk and dv; r_q, r_k, dr_q and dr_k are bf16 either way (the reference
 * asserts bf16 ranks, FNA2/flash_naylis_attn.py:1419-1420, and is generic
 * over the q/k/v dtype, :187, :201, :522-529).  fna2_rope_varlen takes all
 * three; fna2_decode takes bf16. */
enum fna2_dtype { FNA2_BF16 = 1, FNA2_F16 = 2, FNA2_F32 = 3 };

/* Return codes. */
enum fna2_status {
  FNA2_OK = 0,
  FNA2_E_NULL = -1,        /* a required pointer is NULL                     */
  FNA2_E_DTYPE = -2,       /* unsupported element type                       */
  FNA2_E_HEAD_DIM = -3,    /* head_dim not in {64, 128}                      */
  FNA2_E_RANK = -4,        /* rank not a multiple of 8 in [8, 64]            */
  FNA2_E_HEADS = -5,       /* heads / heads_kv / heads_graph inconsistent    */
  FNA2_E_SHAPE = -6,       /* negative or zero-sized extent, or overflow     */
  FNA2_E_STRIDE = -7,      /* stride or pointer not 16-byte aligned          */
  FNA2_E_SEQLENS = -8,     /* varlen without cu_seqlens                      */
  FNA2_E_WORKSPACE = -9,   /* workspace missing or too small                 */
  FNA2_E_LAUNCH = -10,     /* a kernel launch failed                         */
  FNA2_E_DEVICE = -11,     /* current device is not gfx950                   */
  FNA2_E_SCALE = -12,      /* softmax_scale not finite                       */
  FNA2_E_ALIAS = -13,      /* an output overlaps its input without equal it  */
  FNA2_E_SCRATCH = -14     /* beyond fna2_fwd_noalloc's static scratch       */
};

/* A bf16/fp32 tensor view: base pointer + element strides. */
typedef struct fna2_tensor {
  void* ptr;
  int64_t stride_b; /* dense only */
  int64_t stride_s;
  int64_t stride_h;
} fna2_tensor;

/* Problem shape shared by the forward and the backward. */
typedef struct fna2_problem {
  int32_t dtype;       /* enum fna2_dtype */
  int32_t varlen;      /* 0 dense [B,H,S,*], 1 packed [T,H,*] with cu_seqlens */
  int32_t batch;       /* dense: B; varlen: number of sequences N            */
  int32_t seqlen_q;    /* dense: S_q; varlen: max_seqlen_q (a scheduling hint) */
  int32_t seqlen_k;    /* dense: S_k; varlen: max_seqlen_k (a scheduling hint) */
  int32_t total_q;     /* varlen: token count of q/out (bounds every access) */
  int32_t total_k;     /* varlen: token count of k/v                         */
  int32_t heads;       /* H: query heads                                     */
  int32_t heads_kv;    /* H_KV: divides H (GQA)                              */
  int32_t heads_graph; /* H_G <= H: heads [0, H_G) carry the low-rank bias   */
  int32_t head_dim;    /* D in {64, 128}                                     */
  int32_t rank;        /* R: multiple of 8 in [8, 64] (ignored if H_G == 0)  */
  int32_t causal;      /* 1: key j visible to query i iff j <= i             */
  float softmax_scale;
  const int32_t* cu_seqlens_q; /* varlen: [N+1] device int32               */
  const int32_t* cu_seqlens_k; /* varlen: [N+1] device int32               */
} fna2_problem;

typedef struct fna2_fwd_args {
  fna2_problem p;
  fna2_tensor q;   /* [.., H,    D] */
  fna2_tensor k;   /* [.., H_KV, D] */
  fna2_tensor v;   /* [.., H_KV, D] */
  fna2_tensor r_q; /* [.., H_G,  R] */
  fna2_tensor r_k; /* [.., H_G,  R] */
  const float* graph_scale; /* [H_G] fp32 */
  fna2_tensor out; /* [.., H, D], written */
  fna2_tensor lse; /* fp32 [.., H] (feature size 1), written */
  void* workspace;
  size_t workspace_bytes;
  /* Optional (may be NULL): FNA2_FWD_EVENTS hipEvent_t handles owned by the
   * caller; recorded on the stream immediately before and after the
   * attention kernel, for per-kernel timing. */
  void* const* events;
  /* Optional (varlen; may be NULL): a plan buffer of fna2_plan_bytes.  The
   * forward's one list-building launch then also builds the backward's
   * lists into it, and a fna2_bwd given the same plan (and the same
   * problem) launches no builder: one launch fewer per training step. */
  void* plan;
  size_t plan_bytes;
  /* Nonzero: `plan` was filled by an earlier fna2_fwd of this problem with
   * cu_seqlens of unchanged contents (the caller's guarantee; ordered before
   * this call on the stream), so its lists are reused and this call launches
   * no builder (e.g. the layers of one model step, which share cu_seqlens).
   * The library still checks that its record of the plan matches the
   * problem (sizes, causal flag, cu_seqlens pointers, key-tile size) and
   * builds the lists when it does not.  0: build them. */
  int32_t plan_filled;
} fna2_fwd_args;

#define FNA2_FWD_EVENTS 2 /* attention kernel start, end */
#define FNA2_BWD_EVENTS 4 /* dQ start/end, dK-dV start/end */

typedef struct fna2_bwd_args {
  fna2_problem p;
  fna2_tensor q, k, v, r_q, r_k;
  const float* graph_scale;
  fna2_tensor out;   /* forward output                 */
  fna2_tensor lse;   /* forward LSE (fp32)             */
  fna2_tensor dout;  /* upstream gradient, like out    */
  fna2_tensor delta; /* fp32 like lse: sum_d O dO, written */
  fna2_tensor dq;    /* like q,   written              */
  fna2_tensor dk;    /* like k,   written              */
  fna2_tensor dv;    /* like v,   written              */
  fna2_tensor dr_q;  /* like r_q, written              */
  fna2_tensor dr_k;  /* like r_k, written              */
  float* d_graph_scale; /* [H_G] fp32, written         */
  void* workspace;
  size_t workspace_bytes;
  /* Optional (may be NULL): FNA2_BWD_EVENTS hipEvent_t handles owned by the
   * caller, recorded around the dQ/dRq kernel (which also forms delta)
   * and the dK/dV/dRk kernel. */
  void* const* events;
  /* Optional (varlen; may be NULL): the plan a fna2_fwd of the same problem
   * filled.  The dQ kernel's spare workgroups then zero the gradient rows
   * of tokens outside every sequence (the list-building launch does that
   * without a plan).  The library remembers which plans its forwards filled
   * and for which sequences (cu_seqlens pointers, sequence and token counts,
   * causal flag); a plan it did not fill for this problem is ignored, and
   * the backward builds its own lists as without one. */
  const void* plan;
  size_t plan_bytes;
} fna2_bwd_args;

/* Varlen rotary position embedding: positions restart at 0 in every packed
 * sequence.  For token t of sequence b (cu_seqlens[b] <= t < cu_seqlens[b+1]),
 * p = t - cu_seqlens[b], and i < D/2:
 *     angle_i   = p * inv_freq[i]
 *     y_i       = x_i cos(angle_i) - x_{i+D/2} sin(angle_i)
 *     y_{i+D/2} = x_{i+D/2} cos(angle_i) + x_i sin(angle_i)
 * for every head of q and of k, each step rounded to the element type where
 * the reference's eager code rounds (position, inv_freq, angle, cos, sin,
 * each product, the sum).  sign = -1 rotates by -angle_i (the gradient:
 * dx from dy).  Tokens outside [cu_seqlens[0], cu_seqlens[N]) are copied
 * unchanged.  Replaces NaylisAttention._apply_rope_varlen with
 * RotaryPositionalEmbedding.forward (FNA2/attention_fna2.py:620-647,
 * :143-170), which loops over the sequences on the host. */
typedef struct fna2_rope_args {
  int32_t dtype;        /* enum fna2_dtype: q, k, q_out, k_out             */
  int32_t total_tokens; /* T                                               */
  int32_t heads_q;      /* heads of q (0: q absent)                        */
  int32_t heads_k;      /* heads of k (0: k absent)                        */
  int32_t head_dim;     /* D: a power of two in [16, 512]                  */
  int32_t nseq;         /* N >= 0                                          */
  int32_t sign;         /* +1 rotate, -1 rotate back                       */
  const int32_t* cu_seqlens; /* [N+1] device int32, nondecreasing          */
  const float* inv_freq;     /* [D/2] device fp32                           */
  fna2_tensor q, k;          /* [T, heads, D] (stride_s, stride_h)         */
  fna2_tensor q_out, k_out;  /* written; each equal to its input or disjoint */
  /* Optional RMSNorm of every q / k row before the rotation (the reference's
   * q_norm / k_norm, FNA2/attention_fna2.py:95-103, :558-561):
   *     x <- x * rsqrt(mean(x^2) + norm_eps) * norm_[qk]
   * NULL: that side is not normalised.  With a norm the whole chain is
   * evaluated in fp32 and rounded once to the element type. */
  const float* norm_q;       /* [D] fp32 or NULL                           */
  const float* norm_k;       /* [D] fp32 or NULL                           */
  float norm_eps;
} fna2_rope_args;

/* Backward of fna2_rope_varlen: dq and dk from the gradients of q_out and
 * k_out, and (with a norm) the gradients of the norm weights.  Without a
 * norm it is the inverse rotation (no workspace); with one it needs the
 * forward's inputs (fwd.q, fwd.k) and fna2_rope_bwd_workspace_bytes of
 * workspace, and sums the weight gradients in a fixed order. */
typedef struct fna2_rope_bwd_args {
  fna2_rope_args fwd;          /* the forward call's arguments              */
  fna2_tensor dq_out, dk_out;  /* gradients of q_out and k_out              */
  fna2_tensor dq, dk;          /* written (each equal to its gradient input or disjoint) */
  float* dnorm_q;              /* [D] fp32, written when fwd.norm_q is set  */
  float* dnorm_k;              /* [D] fp32, written when fwd.norm_k is set  */
  void* workspace;
  size_t workspace_bytes;
} fna2_rope_bwd_args;

/* Host-only validation of a rotary call (shapes, strides, alignment,
 * aliasing); no GPU call. */
int fna2_check_rope(const fna2_rope_args* args);

/* Rotary embedding of q and k on the stream given (one launch). */
int fna2_rope_varlen(const fna2_rope_args* args, void* hip_stream);

/* Workspace bytes fna2_rope_bwd needs (0 without a norm). */
size_t fna2_rope_bwd_workspace_bytes(const fna2_rope_args* fwd);

/* Host-only validation of a rotary backward call; no GPU call. */
int fna2_check_rope_bwd(const fna2_rope_bwd_args* args);

/* Backward of fna2_rope_varlen (one launch without a norm, two with). */
int fna2_rope_bwd(const fna2_rope_bwd_args* args, void* hip_stream);

/* One-token decode against a KV cache.  Sequence b has one new query row per
 * head and len_b cached rows (the new token's row included), all visible:
 *     S_j = softmax_scale <q_h, K_j> + [h < H_G] graph_scale[h] <rq_h, Rk_hj>
 * for j < len_b, normalised as in fna2_fwd (O = sum e^{S-m} V / (l + 1e-6)).
 * The result equals the last row of the causal fna2_fwd over the sequence.
 * With heads_graph = 0 it is the reference's decode step, which runs PyTorch
 * SDPA over torch.cat(past_kv, new) (FNA2/attention_fna2.py:412-429,
 * :445-473; no graph bias there because no Rk is cached).  Caching Rk
 * (rk_cache) lets a model decode with the bias it was trained with.
 *
 * Layouts (element strides, feature stride 1, rows 16-byte aligned):
 *   q   [B, H, D]          (b, h, f)    at ptr + b*stride_b + h*stride_h + f
 *   r_q [B, H_G, R]        likewise; out [B, H, D] likewise (written)
 *   k_cache, v_cache [B, H_KV, L, D]: (b, h, j, f) at
 *                          ptr + b*stride_b + h*stride_h + j*stride_s + f
 *   rk_cache [B, H_G, L, R] likewise
 *   lse fp32 [B, H]        (b, h) at ptr + b*stride_b + h*stride_h
 * H / H_KV may not exceed 32 (FNA2_E_HEADS: a group's heads are the 32
 * columns of one MFMA tile), and the graph heads of one group times R may
 * not exceed 256 (FNA2_E_RANK).  Byte offsets inside one (b, KV head) -- (H/H_KV - 1) *
 * stride_h + 32 * stride_s of a cache, (H/H_KV - 1) * stride_h of q / r_q,
 * in bytes -- must stay below 2^31 (FNA2_E_SHAPE). */
typedef struct fna2_decode_args {
  int32_t batch;        /* B >= 0                                           */
  int32_t heads;        /* H                                                */
  int32_t heads_kv;     /* H_KV: divides H                                  */
  int32_t heads_graph;  /* H_G <= H (0: no bias; r_q, rk_cache unused)      */
  int32_t head_dim;     /* D in {64, 128}                                   */
  int32_t rank;         /* R: multiple of 8 in [8, 64] (if H_G > 0)         */
  int32_t max_seqlen_k; /* L >= 0: rows each cache holds per (b, head)      */
  int32_t num_splits;   /* key splits per (b, KV head): 0 = library's choice, else 1..64 */
  float softmax_scale;
  const int32_t* seqlens_k; /* [B] device int32 len_b (clamped to [0, L]); NULL: all L */
  fna2_tensor q, r_q;
  fna2_tensor k_cache, v_cache, rk_cache;
  const float* graph_scale; /* [H_G] fp32 */
  fna2_tensor out;          /* written                                      */
  fna2_tensor lse;          /* written; ptr NULL: not computed              */
  void* workspace;          /* fna2_decode_workspace_bytes                  */
  size_t workspace_bytes;
  /* Optional (may be NULL): FNA2_DECODE_EVENTS hipEvent_t handles, recorded
   * around the split kernel. */
  void* const* events;
} fna2_decode_args;

#define FNA2_DECODE_EVENTS 2

/* Host-only validation of a decode call; no GPU call. */
int fna2_check_decode(const fna2_decode_args* args);

/* Key splits the call will use (num_splits, or the library's choice for the
 * current device), or a negative status. */
int fna2_decode_num_splits(const fna2_decode_args* args);

/* Workspace bytes of a decode call (0 with one split). */
size_t fna2_decode_workspace_bytes(const fna2_decode_args* args);

/* Decode: one launch per split set, plus a merge launch with more than one
 * split.  Writes out (and lse). */
int fna2_decode(const fna2_decode_args* args, void* hip_stream);

/* ABI version (FNA2_ABI_VERSION). */
int fna2_version(void);

/* Static text for a status code. */
const char* fna2_status_string(int status);

/* Host-only validation of shapes, strides, alignment and pointers; no GPU
 * call.  Replaces the reference launchers' asserts
 * (FNA2/flash_naylis_attn.py:718-720, :778). */
int fna2_check_fwd(const fna2_fwd_args* args);
int fna2_check_bwd(const fna2_bwd_args* args);

/* Workspace bytes the forward / backward need for this problem. */
size_t fna2_fwd_workspace_bytes(const fna2_problem* p);
size_t fna2_bwd_workspace_bytes(const fna2_problem* p);

/* Bytes of a plan (the varlen tile lists of the forward and the backward:
 * device-built, so no host synchronisation); 0 in dense mode.  No
 * counterpart in the reference, whose varlen grids are (max_seqlen / BLOCK,
 * H, N) with idle programs (FNA2/flash_naylis_attn.py:784, :1281). */
size_t fna2_plan_bytes(const fna2_problem* p);

/* Forward: writes out and lse.
 * Replaces _fna2_forward (FNA2/flash_naylis_attn.py:700-753) and
 * _fna2_forward_varlen (FNA2/flash_naylis_attn.py:756-804). */
int fna2_fwd(const fna2_fwd_args* args, void* hip_stream);

/* Allocation-free forward.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory, or may not (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * is fna2_fwd with the varlen tile list kept in a static device array of
 * fna2_fwd_noalloc_max_bytes() bytes (1 MiB) that the library holds on every
 * GPU it runs on, instead of in args->workspace (ignored; a plan, if given,
 * is used as by fna2_fwd).  Same results as fna2_fwd; the same kernels.
 * Calls no hipMalloc, hipFree or allocating routine.  A problem whose tile
 * list needs more (fna2_fwd_workspace_bytes > the maximum, i.e. more than
 * about 32,000 query tiles: T / 128 + N) returns FNA2_E_SCRATCH.  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other host threads) race and must be serialised by the caller. */
int fna2_fwd_noalloc(const fna2_fwd_args* args, void* hip_stream);

/* Bytes of fna2_fwd_noalloc's static scratch (the largest workspace it
 * stands in for). */
size_t fna2_fwd_noalloc_max_bytes(void);

/* Backward: writes delta, dq, dk, dv, dr_q, dr_k and d_graph_scale
 * (no pre-zeroing needed; no atomics; bitwise deterministic).
 * Replaces _fna2_backward (FNA2/flash_naylis_attn.py:807-892) and
 * _fna2_backward_varlen (FNA2/flash_naylis_attn.py:1215-1300). */
int fna2_bwd(const fna2_bwd_args* args, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* FNA2_H_ */
