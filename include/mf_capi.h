/*
 * mf_capi.h -- C ABI of libmf_hip.so, the MI355X (gfx950) kernels behind
 * Matterformer's geometric-attention hot path.
 *
 * Plain C: device pointers, sizes and an opaque stream handle (a hipStream_t
 * passed as void*; NULL means the legacy default stream).  No C++ or torch
 * types cross this boundary.  Every entry point is stream-ordered and
 * asynchronous: it validates its arguments on the host, enqueues kernels and
 * returns.  The caller owns every buffer; no entry point allocates device
 * memory.
 *
 * Return value: MF_OK (0) or a negative mf_status.  mf_last_error() returns a
 * thread-local, human-readable description of the most recent failure on the
 * calling thread.
 *
 * Scratch device memory an entry point needs is passed in by the caller as a
 * workspace whose size the matching mf_*_workspace_size() reports; the
 * workspace may be reused by later calls on the same stream.
 *
 * Reference interfaces replaced (paths relative to stases/Matterformer):
 *   mf_simplicial_fwd   <- triton_simplicial_attention_forward
 *                          src/matterformer/models/triton_simplicial_attention.py:790-926
 *                          (the launch of _streaming_forward_kernel at :881-922)
 *   mf_knn              <- knn / knn_graph (torch_cluster wrapper with a
 *                          cdist+topk fallback)
 *                          legacy/rapidash_v5/models/rapidash_utils.py:139-193
 *   mf_radius_mask      <- minimum-image pair distance of PeriodicGeometryAdapter.forward
 *                          src/matterformer/geometry/adapters.py:176-190, thresholded
 *   mf_radius_attn      <- masked MHA through an additive attn_mask
 *                          src/matterformer/models/transformer.py:256-268 ->
 *                          src/matterformer/models/regular_attention.py:262-268,303-308
 */
#ifndef MF_CAPI_H
#define MF_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MF_ABI_VERSION 11

typedef enum mf_status {
  MF_OK = 0,
  MF_ERR_INVALID_ARGUMENT = -1, /* null pointer, bad size, bad enum value */
  MF_ERR_UNSUPPORTED = -2,      /* valid request this build cannot serve (e.g. LDS capacity) */
  MF_ERR_HIP = -3               /* a HIP runtime call failed */
} mf_status;

/* Element type of the q/k/v operands. */
typedef enum mf_dtype {
  MF_DTYPE_F32 = 0,
  MF_DTYPE_F16 = 1,
  MF_DTYPE_BF16 = 2
} mf_dtype;

/* Mirrors SUPPORTED_SIMPLICIAL_PRECISIONS = ("bf16_tc", "tf32", "ieee_fp32")
 * (triton_simplicial_attention.py:13).  With 16-bit operands, bf16_tc runs
 * 16-bit MFMA with fp32 accumulation; fp32 operands always run fp32 MFMA. */
typedef enum mf_precision {
  MF_PREC_BF16_TC = 0,
  MF_PREC_TF32 = 1,
  MF_PREC_IEEE_FP32 = 2
} mf_precision;

int mf_abi_version(void);
const char* mf_last_error(void);

/* ------------------------------------------------------------------------ */
/* 2-simplicial attention forward.                                           */
/*                                                                           */
/* For every batch b, head h and valid query i:                              */
/*   S[j,k] = sum_d q[i,d] * k1[j,d] * k2[k,d]                                */
/*   P      = softmax over the valid (j,k) pairs of S                        */
/*   out[i] = sum_{j,k} P[j,k] * (v1[j] (.) v2[k])                           */
/*   lse[i] = log sum_{j,k} exp(S[j,k])                                      */
/* (j,k) is valid iff pair_key_valid[b,j] && pair_key_valid[b,k] &&          */
/* (pair_valid == NULL || pair_valid[b,j,k]).  Rows of invalid queries, and  */
/* queries with no valid pair, get out = 0 and lse = 0.                      */
/* Semantics follow simplicial_attention.py:206-344 and                      */
/* triton_simplicial_attention.py:115-329.                                   */
/* ------------------------------------------------------------------------ */
typedef struct mf_simplicial_fwd_args {
  /* [B*H, N, D] contiguous, element type `dtype`. */
  const void* q;
  const void* k1;
  const void* v1;
  const void* k2;
  const void* v2;
  /* [B, N] bytes, nonzero = valid. */
  const uint8_t* query_valid;
  const uint8_t* pair_key_valid;
  /* [B, N, N] bytes or NULL. */
  const uint8_t* pair_valid;
  /* Outputs; any may be NULL but not all three.                              */
  void* out;        /* [B*H, N, D] in `dtype` (the `out.to(q.dtype)` result) */
  float* out_f32;   /* [B*H, N, D] fp32 (the saved-for-backward output)      */
  float* lse;       /* [B*H, N] fp32, natural log                            */
  /* Device scratch of at least mf_simplicial_fwd_workspace_size() bytes,
   * 16-byte aligned (NULL when that size is 0).  ZERO IT ONCE before its
   * first use: its first 256 bytes hold the pair kernel's unit-claim
   * counter, which every call leaves at 0 again (graph replays included);
   * the rest holds the other 16-bit kernel's per-call atom lists and work
   * items.  Calls that share a workspace must be ordered on one stream. */
  void* workspace;
  uint64_t workspace_bytes;
  int32_t batch;
  int32_t heads;
  int32_t tokens;
  int32_t head_dim; /* 1..128 */
  int32_t dtype;     /* mf_dtype */
  int32_t precision; /* mf_precision */
  /* Optional logit and message terms; each group is absent when its first
   * pointer is NULL.  Semantics of SimplicialFactorizedBias,
   * SimplicialLowRankAngleResidual and SimplicialLowRankMessageResidual
   * (simplicial_attention.py:18-104,330-337; triton_simplicial_attention.py:
   * 244-279,305-326), with (j,k) valid as above:
   *   factorized bias:  S[j,k] += gate_i * ((u[i,j] + v[i,k]) + w[j,k])
   *   low-rank angle:   S[j,k] += angle_gate_i * Ra^-1/2 * sum_r AL[i,j,r] AR[i,k,r]
   *   low-rank message: out_i  += sum_r c_r basis[h,r,:],
   *                     c_r = Rm^-1/2 * sum_{j,k} P[j,k] ML[i,j,r] MR[i,k,r]
   * (P the normalised softmax weights).  Calls with any of them run the
   * general kernel. */
  const void* bias_u;     /* [B*H, N, N] in bias_dtype                     */
  const void* bias_v;     /* [B*H, N, N]                                   */
  const void* bias_w;     /* [B*H, N, N]                                   */
  const void* bias_gate;  /* [B*H, N]                                      */
  int32_t bias_dtype;     /* mf_dtype of the four bias tensors             */
  int32_t angle_rank;     /* Ra, 1..64 when angle_left != NULL            */
  const float* angle_left;   /* [B*H, N, N, Ra] fp32                       */
  const float* angle_right;  /* [B*H, N, N, Ra] fp32                       */
  const float* angle_gate;   /* [B*H, N] fp32                              */
  const float* message_left;   /* [B*H, N, N, Rm] fp32                     */
  const float* message_right;  /* [B*H, N, N, Rm] fp32                     */
  const float* message_basis;  /* [H, Rm, D] fp32                          */
  int32_t message_rank;        /* Rm, 1..64 when message_left != NULL     */
  /* ABI 8: strides, in elements, of the [B, H, N, D] operands as
   * {batch, head, token} (d is unit-stride), for views such as the chunks of
   * an in_proj output [B, N, 5, H, D] (the reference's _split_heads,
   * simplicial_attention.py:708-711, without its .contiguous() copies) and an
   * out that is the merged [B, N, H, D] layout out_proj reads
   * (_merge_heads).  All three zero: the contiguous [B*H, N, D] layout.
   * Other strides are taken by the pair kernel only (16-bit operands,
   * head_dim <= 64 and a multiple of 8, tokens <= 512, no pair_valid, no
   * angle or message term, every stride a multiple of 8 and below 2^31, every
   * base 16-byte aligned);
   * calls outside that return MF_ERR_UNSUPPORTED.  out_f32 and lse stay
   * contiguous. */
  int64_t q_stride[3];   /* of q                                          */
  int64_t kv_stride[3];  /* shared by k1, v1, k2 and v2                   */
  int64_t out_stride[3]; /* of out                                        */
} mf_simplicial_fwd_args;

int mf_simplicial_fwd(const mf_simplicial_fwd_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* 2-simplicial attention backward (deterministic).                          */
/*                                                                           */
/* With P[i,j,k] = exp(S[i,j,k] - lse[i]) on valid pairs (S including the    */
/* factorized bias when given), go = grad_out and                            */
/* dS[i,j,k] = P[i,j,k] (sum_d go[i,d] v1[j,d] v2[k,d] - go[i] . out[i]):    */
/*   dq[i]  = sum_jk dS k1[j] (.) k2[k]    dk1[j] = sum_ik dS q[i] (.) k2[k]  */
/*   dk2[k] = sum_ij dS q[i] (.) k1[j]     dv1[j] = sum_ik P go[i] (.) v2[k]  */
/*   dv2[k] = sum_ij P go[i] (.) v1[j]                                        */
/*   du[i,j] = gate_i sum_k dS   dv_bias[i,k] = gate_i sum_j dS              */
/*   dw[j,k] = sum_i gate_i dS   dgate[i] = sum_jk dS (u_ij + v_ik + w_jk)   */
/* (the quantities of triton_simplicial_attention.py:332-782 and             */
/* :929-1204, which accumulates them with atomics).  Every output element is */
/* written by one wave after sums in a fixed order: two calls on the same    */
/* inputs give bitwise identical gradients.  dq, dk1, dv1, dk2 and dv2 are  */
/* fp32 (grads_dtype MF_DTYPE_F32), written only at valid entries, the      */
/* caller zero-filling them; or (ABI 10) bf16 when grads_dtype, dtype and   */
/* grad_dtype are all MF_DTYPE_BF16, no low-rank term is given, head_dim is */
/* a multiple of 8, tokens <= 4096 and the buffers are 16-byte aligned: then */
/* every row is written (zeros at padded queries and keys) and the caller   */
/* needs no fill.  The bias gradients follow (ABI 11): fp32, zero-filled   */
/* by the caller and written at valid entries, with grads_dtype F32; bf16,  */
/* every element written (zeros where an index is padded), with grads_dtype */
/* BF16 (16-byte aligned buffers).                                          */
/* With the low-rank terms of mf_simplicial_fwd (angle A_ijk = sum_r         */
/* AL[i,j,r] AR[i,k,r] added to S as ag_i Ra^-1/2 A; message                 */
/* c_ir = Rm^-1/2 sum_jk P ML[i,j,r] MR[i,k,r], out_i += sum_r c_ir          */
/* basis[h,r]), dP gains Rm^-1/2 sum_r dc_ir ML MR with dc_ir = basis[h,r].go_i */
/* and, with sa = Ra^-1/2, sm = Rm^-1/2:                                     */
/*   dangle_left[i,j]  = ag_i sa sum_k dS AR[i,k]                            */
/*   dangle_right[i,k] = ag_i sa sum_j dS AL[i,j]                            */
/*   dangle_gate[i]    = sa sum_jk dS A_ijk                                  */
/*   dmessage_left[i,j]  = sm dc_i (.) sum_k P MR[i,k]                       */
/*   dmessage_right[i,k] = sm dc_i (.) sum_j P ML[i,j]                       */
/*   dmessage_basis[h,r] = sm sum_(b,i valid) (sum_jk P ML MR)_ir go_i       */
/* (triton_simplicial_attention.py:488-515,575-782).  Calls with these       */
/* terms run fp32 arithmetic for every operand dtype.                        */
/* Replaces triton_simplicial_attention_backward,                            */
/* triton_simplicial_attention.py:929-1204.                                  */
/* ------------------------------------------------------------------------ */
typedef struct mf_simplicial_bwd_args {
  const void* q;            /* [B*H, N, D] element type `dtype`              */
  const void* k1;
  const void* v1;
  const void* k2;
  const void* v2;
  const void* grad_out;     /* [B*H, N, D] element type `grad_dtype`         */
  const float* out;         /* [B*H, N, D] fp32 forward output (out_f32)     */
  const float* lse;         /* [B*H, N] fp32 forward lse                     */
  const uint8_t* query_valid;     /* [B, N]                                  */
  const uint8_t* pair_key_valid;  /* [B, N]                                  */
  const uint8_t* pair_valid;      /* [B, N, N] or NULL                       */
  const void* bias_u;       /* factorized bias as in mf_simplicial_fwd, or NULL */
  const void* bias_v;
  const void* bias_w;
  const void* bias_gate;
  int32_t bias_dtype;
  int32_t grad_dtype;       /* mf_dtype of grad_out                          */
  void* dq;                 /* [B*H, N, D] each, type `grads_dtype`; NULL = not wanted */
  void* dk1;
  void* dv1;
  void* dk2;
  void* dv2;
  void* du;                 /* [B*H, N, N] each, type `grads_dtype` (bias only); NULL = not wanted */
  void* dv_bias;
  void* dw;
  void* dgate;              /* [B*H, N], type `grads_dtype`                   */
  int32_t batch;
  int32_t heads;
  int32_t tokens;
  int32_t head_dim;         /* 1..128                                        */
  int32_t dtype;            /* mf_dtype of q, k1, v1, k2, v2                 */
  int32_t grads_dtype;      /* ABI 10: MF_DTYPE_F32 (0) or MF_DTYPE_BF16     */
  /* Low-rank angle and message terms (ABI 9), laid out as in              */
  /* mf_simplicial_fwd_args; a group is absent when its first pointer is   */
  /* NULL.  Their gradients are fp32, zero-filled by the caller, written   */
  /* only at valid entries; NULL = not wanted.                             */
  int32_t angle_rank;           /* Ra, 1..64 when angle_left != NULL       */
  int32_t message_rank;         /* Rm, 1..64 when message_left != NULL     */
  const float* angle_left;      /* [B*H, N, N, Ra] fp32                    */
  const float* angle_right;     /* [B*H, N, N, Ra] fp32                    */
  const float* angle_gate;      /* [B*H, N] fp32                           */
  const float* message_left;    /* [B*H, N, N, Rm] fp32                    */
  const float* message_right;   /* [B*H, N, N, Rm] fp32                    */
  const float* message_basis;   /* [H, Rm, D] fp32                         */
  float* dangle_left;           /* [B*H, N, N, Ra]                         */
  float* dangle_right;          /* [B*H, N, N, Ra]                         */
  float* dangle_gate;           /* [B*H, N]                                */
  float* dmessage_left;         /* [B*H, N, N, Rm]                         */
  float* dmessage_right;        /* [B*H, N, N, Rm]                         */
  float* dmessage_basis;        /* [H, Rm, D]                              */
  void* workspace;              /* mf_simplicial_bwd_workspace_size() bytes (NULL when 0) */
  uint64_t workspace_bytes;
} mf_simplicial_bwd_args;

int mf_simplicial_bwd(const mf_simplicial_bwd_args* args, void* stream);

/* Bytes of workspace mf_simplicial_bwd needs (0 without a message term):   */
/* per query, the message coefficients dc = basis . go and sum_jk P ML MR.  */
uint64_t mf_simplicial_bwd_workspace_size(int32_t batch, int32_t heads, int32_t tokens,
                                          int32_t head_dim, int32_t message_rank);

/* Returns MF_OK when mf_simplicial_fwd can serve this shape on the current
 * device, MF_ERR_UNSUPPORTED (with mf_last_error set) when it cannot. */
int mf_simplicial_fwd_supported(int32_t batch, int32_t heads, int32_t tokens,
                                int32_t head_dim, int32_t dtype);

/* Bytes of workspace mf_simplicial_fwd needs for this shape (0 if none). */
uint64_t mf_simplicial_fwd_workspace_size(int32_t batch, int32_t heads, int32_t tokens,
                                          int32_t head_dim, int32_t dtype);

/* Allocation-free variant of mf_simplicial_fwd.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, validation and results as mf_simplicial_fwd, except that
 * `workspace` and `workspace_bytes` are ignored: the scratch lives in a static
 * 8 MiB device array, one per GPU, held until the process ends.  A shape whose
 * mf_simplicial_fwd_workspace_size() exceeds 8 MiB returns MF_ERR_UNSUPPORTED.
 * The call allocates nothing (no hipMalloc/hipFree, no allocating library
 * routine).  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (two streams, concurrent graph replays) race. */
int mf_simplicial_fwd_noalloc(const mf_simplicial_fwd_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* k nearest neighbours of every atom of a batch of molecules.               */
/*                                                                           */
/* Distance convention of NonPeriodicGeometryAdapter.forward                 */
/* (geometry/adapters.py:98-100): delta = x_i - x_j,                         */
/* d2 = (dx*dx + dy*dy) + dz*dz in fp32, each operation rounded (no FMA).    */
/* For every valid atom i the k valid atoms j (j != i when exclude_self)     */
/* with the smallest (d2, j) -- ties go to the lower index -- in ascending   */
/* order; dist = sqrt(d2) correctly rounded.  Slots beyond the number of     */
/* candidates, and every slot of a padded atom, get idx -1 and dist +inf.    */
/* Replaces the legacy knn / knn_graph (cdist + topk, unspecified tie order) */
/* of legacy/rapidash_v5/models/rapidash_utils.py:139-193.                   */
/* ------------------------------------------------------------------------ */
typedef struct mf_knn_args {
  const float* coords;     /* [B, N, 3] fp32, finite                         */
  const uint8_t* pad_mask; /* [B, N] bytes, nonzero = padding, or NULL       */
  int32_t* idx;            /* [B, N, k] out                                  */
  float* dist;             /* [B, N, k] out, or NULL                         */
  int32_t batch;
  int32_t atoms;           /* N >= 1                                         */
  int32_t k;               /* 1 <= k <= 64                                   */
  int32_t exclude_self;    /* nonzero: j == i is not a candidate             */
} mf_knn_args;

int mf_knn(const mf_knn_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* kNN lists -> local-attention masks in the layout mf_radius_attn reads.    */
/*                                                                           */
/*   mask[b,i,j] = valid_i && (j in idx[b,i,:] || (include_self && j == i))  */
/* mask_bits [B, N, ceil(N/32)] (bit t of word w is column 32w+t, columns    */
/* >= N are 0) and block_mask [B, NB, NB] for 64-atom tiles (NB = ceil(N/64)) */
/* as mf_radius_mask writes them.  The reference has no kNN attention; its   */
/* trunk expresses one only as MHA with a 0/-inf attn_head_bias              */
/* (src/matterformer/models/transformer.py:256-268), whose allowed entries   */
/* are these bits.                                                           */
/* ------------------------------------------------------------------------ */
typedef struct mf_knn_mask_args {
  const int32_t* idx;      /* [B, N, k] as mf_knn writes it (-1 = none)     */
  const uint8_t* pad_mask; /* [B, N] bytes, nonzero = padding, or NULL       */
  uint32_t* mask_bits;     /* out                                            */
  uint8_t* block_mask;     /* out, or NULL                                   */
  int32_t batch;
  int32_t atoms;
  int32_t k;
  int32_t include_self;    /* nonzero: every valid atom is its own neighbour */
} mf_knn_mask_args;

int mf_knn_mask(const mf_knn_mask_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Cutoff (radius) neighbour mask, minimum image for periodic cells.         */
/*                                                                           */
/* periodic (gram != NULL): coords are fractional; for the integer image     */
/*   offsets o in {-r..r}^3 (r = pbc_radius, PeriodicGeometryAdapter,        */
/*   adapters.py:141-149,176-190), e = (f_i - f_j) + o and                   */
/*   t_c = (G[c][0]*e0 + G[c][1]*e1) + G[c][2]*e2,                          */
/*   d2  = (e0*t0 + e1*t1) + e2*t2, minimised over the images;               */
/* non-periodic (gram == NULL): d2 = (dx*dx + dy*dy) + dz*dz (adapters.py:98-99). */
/* fp32, each operation rounded.  mask[i,j] = d2 <= cutoff*cutoff for valid  */
/* i and j (i == j included).                                                */
/*   mask_bits  [B, N, ceil(N/32)] uint32: bit t of word w is column 32w+t;  */
/*              bits of columns >= N are 0.                                  */
/*   block_mask [B, NB, NB] bytes (NB = ceil(N/block)), or NULL: 1 iff any   */
/*              bit of the (block x block) tile is set.                      */
/* block is 32, 64 or 128.                                                   */
/* ------------------------------------------------------------------------ */
typedef struct mf_radius_mask_args {
  const float* coords;     /* [B, N, 3] fp32 (fractional when periodic)      */
  const float* gram;       /* [B, 3, 3] fp32 metric G = cell cell^T, or NULL */
  const uint8_t* pad_mask; /* [B, N] bytes, nonzero = padding, or NULL       */
  uint32_t* mask_bits;     /* out                                            */
  uint8_t* block_mask;     /* out, or NULL                                   */
  float cutoff;            /* > 0                                            */
  int32_t batch;
  int32_t atoms;
  int32_t block;
  int32_t pbc_radius;      /* 1 or 2 (ignored when gram == NULL)             */
} mf_radius_mask_args;

int mf_radius_mask(const mf_radius_mask_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Pairwise geometry features in one pass, optionally with the cutoff mask. */
/*                                                                           */
/* The pair tensors of GeometryFeatures (geometry/adapters.py:12-21) as the  */
/* adapters compute them:                                                    */
/*   gram == NULL (NonPeriodicGeometryAdapter.forward, adapters.py:83-125):  */
/*     delta = x_i - x_j, d2 = (dx*dx + dy*dy) + dz*dz;                      */
/*   gram != NULL (PeriodicGeometryAdapter.forward, adapters.py:151-212):    */
/*     coords fractional; delta = (f_i - f_j) + o for the first offset o of  */
/*     {-r..r}^3 (itertools.product order) minimising d2 = e^T G e, with     */
/*     d2 evaluated as in mf_radius_mask;                                    */
/*   d2 = max(d2, 0), dist = sqrt(d2), dist_norm = dist / scale[b].          */
/* Every output is 0 outside the valid pairs (both atoms valid).  mask_bits, */
/* when given, are mf_radius_mask's bits for `cutoff` (d2 <= cutoff^2 on    */
/* valid pairs, i == j included), in its layout.  Replaces the               */
/* [B, N, N, 27, 3] image tensor of adapters.py:176-189.                     */
/* ------------------------------------------------------------------------ */
typedef struct mf_geometry_args {
  const float* coords;     /* [B, N, 3] fp32 (fractional when periodic)      */
  const float* gram;       /* [B, 3, 3] fp32 metric, or NULL (non-periodic)  */
  float* scale;            /* [B] fp32 normaliser of dist_norm, or NULL; read
                              (MF_SCALE_GIVEN) or written first (MF_SCALE_RMS) */
  const uint8_t* pad_mask; /* [B, N] bytes, nonzero = padding, or NULL       */
  float* pair_delta;       /* [B, N, N, 3] out, or NULL                      */
  float* pair_dist2;       /* [B, N, N] out, or NULL                         */
  float* pair_dist;        /* [B, N, N] out, or NULL                         */
  float* pair_dist_norm;   /* [B, N, N] out (needs scale), or NULL           */
  uint32_t* mask_bits;     /* [B, N, ceil(N/32)] out, or NULL                */
  float cutoff;            /* > 0 when mask_bits is given                    */
  int32_t batch;
  int32_t atoms;
  int32_t pbc_radius;      /* 1 or 2 (ignored when gram == NULL)             */
  /* ABI 7: the adapter's small steps in the same call                        */
  uint8_t* pair_mask;      /* [B, N, N] out: 1 on valid pairs, or NULL       */
  int32_t scale_mode;      /* MF_SCALE_GIVEN: read `scale`; MF_SCALE_RMS:
                              write the root-mean-square |x| of each molecule's
                              valid atoms (the non-periodic adapter's radius,
                              adapters.py:116-118) into `scale`, then use it */
} mf_geometry_args;

#define MF_SCALE_GIVEN 0
#define MF_SCALE_RMS 1

int mf_geometry_features(const mf_geometry_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* The lattice terms of the periodic adapter in one launch (ABI 11).         */
/*                                                                           */
/* For a batch of lattice latents [B, 6] fp32 in `lattice_repr`:             */
/*   gram[b]       = C C^T of the lower-triangular cell C (the metric),      */
/*                   non-finite entries replaced by 0                        */
/*                   (lattice_latent_to_gram, geometry/lattice.py:12-59,94-100); */
/*   y1[b]         = the clamped y1 latent (y1), or y1 recovered from gram   */
/*                   (ltri) (lattice_latent_to_y1, lattice.py:65-91,103-131); */
/*   cell_scale[b] = max(mean(exp(y1[b, 0:3])), 1e-8)                        */
/*                   (PeriodicGeometryAdapter.forward, adapters.py:173-174,192). */
/* Each output may be NULL.  fp32 throughout, every operation rounded as the */
/* torch formulation evaluates it.  Replaces the ~27 small torch kernels of  */
/* those three lines on a [B, 6] tensor.                                      */
/* ------------------------------------------------------------------------ */
#define MF_LATTICE_Y1 0
#define MF_LATTICE_LTRI 1

int mf_lattice_terms(const float* lattice, int32_t batch, int32_t lattice_repr, float* gram, float* y1,
                     float* cell_scale, void* stream);

/* ------------------------------------------------------------------------ */
/* Local (radius) attention over a neighbour bit mask.                        */
/*                                                                           */
/* out[b,h,i] = sum_j softmax_j(scale * q_i . k_j over j with mask[b,i,j]) v_j */
/* lse[b,h,i] = log sum_j exp(scale * q_i . k_j) over the same j; rows with  */
/* no allowed key get out = 0 and lse = 0.  This is the dense masked softmax */
/* that an additive attn_mask (0 / -inf) gives in nn.MultiheadAttention and  */
/* scaled_dot_product_attention (transformer.py:256-268,                     */
/* regular_attention.py:262-268,303-308), skipping 64x64 tiles whose         */
/* block_mask entry is 0.                                                    */
/* ------------------------------------------------------------------------ */
typedef struct mf_radius_attn_args {
  const void* q;               /* [B, H, N, D], dtype bf16 or fp16           */
  const void* k;
  const void* v;
  const uint32_t* mask_bits;   /* [B, N, ceil(N/32)] as mf_radius_mask writes */
  const uint8_t* block_mask;   /* [B, NB, NB] for block 64, or NULL (all tiles) */
  void* out;                   /* [B, H, N, D] dtype, or NULL                */
  float* out_f32;              /* [B, H, N, D] fp32, or NULL                 */
  float* lse;                  /* [B, H, N] fp32 (natural log), or NULL      */
  float scale;                 /* logit scale, e.g. head_dim^-1/2            */
  int32_t batch;
  int32_t heads;
  int32_t atoms;
  int32_t head_dim;            /* 32, 64 or 128                              */
  int32_t dtype;               /* MF_DTYPE_BF16 or MF_DTYPE_F16              */
} mf_radius_attn_args;

int mf_radius_attn(const mf_radius_attn_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Packed-token glue of the AdaLN trunk.  The valid atoms of a padded batch  */
/* are the T rows of one [T, C] matrix (row t: atom of molecule mol[t]).     */
/* All three replace torch expressions of the reference's AdaLNBlock and     */
/* SimplicialAttention; none has a kernel of its own in the reference.       */
/*                                                                           */
/* mf_adaln_rows: the elementwise steps around a block's attention and MLP   */
/* (transformer.py:296-316, _modulate):                                      */
/*   y != NULL:     x_out = x + gate[mol] * y                                */
/*   shift != NULL: h_out = LN(x') * (1 + scale[mol]) + shift[mol],          */
/*                  x' = x_out if y != NULL else x; LN without affine, eps.  */
/* Every product and sum rounded to dtype as the torch expressions are; LN  */
/* statistics in fp32.  x_out may equal x.  channels and mod_stride multiples */
/* of 8, channels <= 2048, operands 16-byte aligned (else                    */
/* MF_ERR_UNSUPPORTED).                                                      */
/* ------------------------------------------------------------------------ */
typedef struct mf_adaln_rows_args {
  const void* x;           /* [T, C] residual stream                          */
  const void* y;           /* [T, C] branch output, or NULL                   */
  const void* gate;        /* [B, .] row stride mod_stride (with y)           */
  const void* shift;       /* [B, .] row stride mod_stride, or NULL           */
  const void* scale;       /* [B, .] row stride mod_stride (with shift)       */
  const int32_t* mol;      /* [T] molecule of each row                        */
  void* x_out;             /* [T, C] (with y)                                 */
  void* h_out;             /* [T, C] (with shift)                             */
  float eps;
  int32_t tokens;
  int32_t channels;
  int32_t batch;
  int32_t mod_stride;      /* elements between molecules' gate/shift/scale rows */
  int32_t dtype;           /* mf_dtype of every tensor                        */
} mf_adaln_rows_args;

int mf_adaln_rows(const mf_adaln_rows_args* args, void* stream);

/* mf_rows_to_heads: [T, P*H*D] projections (in_proj output, parts q/k/v...) */
/* -> [P, B, H, W, D], the layout the attention kernels read:                 */
/*   heads[p, b, h, w, :] = rows[slot[b*W + w], p*H*D + h*D : +D]             */
/* (zeros where slot is -1); part 0 multiplied by first_part_scale and       */
/* rounded in the source dtype first (q * head_dim^-1/2, _project_inputs),   */
/* then converted to dst_dtype.  D multiple of 8, 16-byte aligned operands.  */
typedef struct mf_rows_to_heads_args {
  const void* rows;        /* [T, P*H*D] src_dtype                            */
  const int32_t* slot;     /* [B*W]: source row of (b, w), or -1              */
  void* heads;             /* [P, B, H, W, D] dst_dtype                       */
  float first_part_scale;  /* 1 = none                                       */
  int32_t tokens;
  int32_t parts;
  int32_t batch;
  int32_t heads_count;
  int32_t width;           /* W: padded atoms per molecule                    */
  int32_t head_dim;
  int32_t src_dtype;
  int32_t dst_dtype;
} mf_rows_to_heads_args;

int mf_rows_to_heads(const mf_rows_to_heads_args* args, void* stream);

/* mf_heads_to_rows: [B, H, W, D] attention output -> [T, H*D] rows          */
/* (_merge_heads on the valid atoms): rows[t, h*D + d] = heads[b, h, w, d]   */
/* with b*W + w = row_index[t]; converted to dst_dtype.                      */
typedef struct mf_heads_to_rows_args {
  const void* heads;       /* [B, H, W, D] src_dtype                          */
  const int32_t* row_index;/* [T]: b*W + w of row t                          */
  void* rows;              /* [T, H*D] dst_dtype                              */
  int32_t tokens;
  int32_t batch;
  int32_t heads_count;
  int32_t width;
  int32_t head_dim;
  int32_t src_dtype;
  int32_t dst_dtype;
} mf_heads_to_rows_args;

int mf_heads_to_rows(const mf_heads_to_rows_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Factorized simplicial geometry bias from the adapters' pair features      */
/* (SimplicialGeometryBias._compute_factorized_terms, transformer.py:702-717, */
/* with the MLPs of :566-584 and the rbf of :637-640):                        */
/*   spoke x_s = [delta (3), rbf(d_norm) (R)],  pair x_p = rbf(d_norm),       */
/*   rbf_r(x)  = exp(-gamma (x - c_r)^2),                                     */
/*   u = MLP_u(x_s), v = MLP_v(x_s), w = MLP_w(x_p),                          */
/*   MLP(x)    = W2 SiLU(W1 x + b1) + b2   (H outputs),                       */
/* written as [B, H, N, N] fp32 with the diagonal and the pairs outside      */
/* pair_mask zero.  W1 [hidden, F] row-major (F = 3 + R or R, + the periodic */
/* features below), W2 [H, hidden].  fp32 throughout (fp32 MFMA).  R <= 29,  */
/* hidden a multiple of 16 <= 256, H <= 16; periodic spoke features <= 80.  */
/* ------------------------------------------------------------------------ */
typedef struct mf_pair_mlp_args {
  const float* pair_delta;      /* [B, N, N, 3]                               */
  const float* pair_dist_norm;  /* [B, N, N]                                  */
  const uint8_t* pair_mask;     /* [B, N, N] bytes, nonzero = valid pair      */
  const float* rbf_centers;     /* [R]                                        */
  float rbf_gamma;
  const float* u_w1;            /* [hidden, 3 + R] */
  const float* u_b1;            /* [hidden]        */
  const float* u_w2;            /* [H, hidden]     */
  const float* u_b2;            /* [H]             */
  const float* v_w1;
  const float* v_b1;
  const float* v_w2;
  const float* v_b2;
  const float* w_w1;            /* [hidden, R]     */
  const float* w_b1;
  const float* w_w2;
  const float* w_b2;
  float* u_out;                 /* [B, H, N, N]    */
  float* v_out;
  float* w_out;
  int32_t batch;
  int32_t atoms;
  int32_t rbf;
  int32_t hidden;
  int32_t heads;
  /* ABI 11: the periodic features of use_periodic_features (transformer.py:641-652), forward only: the  */
  /* spoke input gains, for each delta component c, sin and cos of (2 pi delta_c) freqs[k] (k < n_freqs), */
  /* then global_geom[b] (6); the pair input gains global_geom[b].  n_freqs = 0 and NULLs: none.          */
  int32_t n_freqs;
  const float* freqs;           /* [n_freqs]       */
  const float* global_geom;     /* [B, 6]          */
} mf_pair_mlp_args;

int mf_pair_mlp_bias(const mf_pair_mlp_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Its backward with respect to the MLP weights (ABI 11), the gradients     */
/* autograd gives SimplicialGeometryBias's u, v, w MLPs (transformer.py:     */
/* 566-584,702-717) for upstream gradients u_grad, v_grad, w_grad of the     */
/* masked outputs (pairs outside pair_mask and the diagonal contribute       */
/* nothing, as the reference's `* mask` makes them):                         */
/*   dW2 = sum_p dY h^T,  db2 = sum_p dY,  dW1 = sum_p dA x^T,  db1 = sum_p dA, */
/*   h = SiLU(W1 x + b1),  dA = (W2^T dY) (.) SiLU'(W1 x + b1).               */
/* `fwd` holds the forward's features and weights (its u_out, v_out, w_out   */
/* are not used).  The features take no gradient.  fp32 MFMA; every sum in  */
/* a fixed order (two calls give identical bits).  R <= 28, hidden a         */
/* multiple of 16 <= 128, H <= 16; the workspace holds per-wave partial sums */
/* (mf_pair_mlp_bias_bwd_workspace_size(hidden) bytes, no fill needed).      */
/* ------------------------------------------------------------------------ */
typedef struct mf_pair_mlp_bwd_args {
  mf_pair_mlp_args fwd;
  const float* u_grad;          /* [B, H, N, N] */
  const float* v_grad;
  const float* w_grad;
  float* u_dw1;                 /* [hidden, 3 + R] */
  float* u_db1;                 /* [hidden]        */
  float* u_dw2;                 /* [H, hidden]     */
  float* u_db2;                 /* [H]             */
  float* v_dw1;
  float* v_db1;
  float* v_dw2;
  float* v_db2;
  float* w_dw1;                 /* [hidden, R]     */
  float* w_db1;
  float* w_dw2;
  float* w_db2;
  void* workspace;
  uint64_t workspace_bytes;
} mf_pair_mlp_bwd_args;

uint64_t mf_pair_mlp_bias_bwd_workspace_size(int32_t hidden);
int mf_pair_mlp_bias_bwd(const mf_pair_mlp_bwd_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MF_CAPI_H */
