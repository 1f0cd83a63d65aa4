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

#define MF_ABI_VERSION 2

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
   * 16-byte aligned (NULL when that size is 0).  Holds the per-molecule
   * atom lists and the work items built on the device for this call. */
  void* workspace;
  uint64_t workspace_bytes;
  int32_t batch;
  int32_t heads;
  int32_t tokens;
  int32_t head_dim; /* 1..128 */
  int32_t dtype;     /* mf_dtype */
  int32_t precision; /* mf_precision */
} mf_simplicial_fwd_args;

int mf_simplicial_fwd(const mf_simplicial_fwd_args* args, void* stream);

/* Returns MF_OK when mf_simplicial_fwd can serve this shape on the current
 * device, MF_ERR_UNSUPPORTED (with mf_last_error set) when it cannot. */
int mf_simplicial_fwd_supported(int32_t batch, int32_t heads, int32_t tokens,
                                int32_t head_dim, int32_t dtype);

/* Bytes of workspace mf_simplicial_fwd needs for this shape (0 if none). */
uint64_t mf_simplicial_fwd_workspace_size(int32_t batch, int32_t heads, int32_t tokens,
                                          int32_t head_dim, int32_t dtype);

#ifdef __cplusplus
}
#endif

#endif /* MF_CAPI_H */
