/*
 * omnimem_hip.h -- C ABI of the MI355X (gfx950) native-sparse-attention selection path.
 *
 * Every entry point takes plain device pointers, element strides and sizes, runs on the HIP
 * stream it is given (passed as void*, a hipStream_t), never synchronises, and returns an
 * OMM_* status.  On failure omm_last_error() returns a thread-local message.  No entry point
 * allocates device memory: scratch is passed in by the caller (see the *_workspace_bytes
 * queries), so a caller's caching allocator owns every byte.
 *
 * Reference interfaces replaced (wuyushuwys/OmniMem, src/omnimem/nsa/...):
 *   omm_block_pool          <- K mean-pool `roped_key.view(b, s//BS, BS, n, d).mean(2)`
 *                              (models/transformers/causal_wan_nsa_model.py:408,481) and the
 *                              query-group pool `q.reshape(B,T//G,G,H,K).mean(2)`
 *                              (nsa/ops/index_topk.py:76)
 *   omm_topk                <- torch.ops.omnimem_nsa.topk (cuda_backend/csrc/bindings.cpp:9-11,
 *                              cuda_backend/csrc/ops.h:11-17, cuda_backend/csrc/topk.cu:664-808)
 *   omm_topk_fused          <- parallel_nsa_topk's query-group pool + the topk op
 *                              (nsa/ops/index_topk.py:72-105 then topk.cu:664-808) in one pass
 *   omm_topk_from_scores    <- the selection half of the same op (topk.cu:366-438): block scores
 *                              in, indices out, so bit-exactness is testable on identical scores
 *   omm_sel_fwd             <- torch.ops.omnimem_nsa.sel_fwd (bindings.cpp:16-19, ops.h:25-29,
 *                              selection_fwd.cu:934-966)
 *   omm_sel_fwd_ptr         <- torch.ops.omnimem_nsa.sel_fwd_ptr (bindings.cpp:20-23,
 *                              selection_fwd.cu:968-992)
 *   omm_sel_fwd_paged       <- selection_attention_padded_ptr_fast
 *                              (nsa/ops/selection/padded_ptr/wrapper.py:458-553) over the paged
 *                              cache, with int32 unit slots instead of raw int64 addresses
 */
#ifndef OMNIMEM_HIP_H_
#define OMNIMEM_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- element types ------------------------------------------------------------------- */
enum {
  OMM_F32 = 0,
  OMM_BF16 = 1,
  OMM_F16 = 2,
  OMM_FP8E4M3 = 3 /* OCP e4m3fn (max 448), cache pages only */
};

/* ---- status codes -------------------------------------------------------------------- */
enum {
  OMM_OK = 0,
  OMM_EINVAL = 1,      /* bad argument: shape, stride, dtype or range */
  OMM_EUNSUPPORTED = 2, /* valid but not implemented (e.g. head dim > 256) */
  OMM_EWORKSPACE = 3,  /* workspace missing or too small */
  OMM_EHIP = 4         /* a HIP launch or runtime call failed */
};

/* [d0, d1, d2, d3] strided view; strides are in elements, sizes and strides >= 0. */
typedef struct omm_view4 {
  const void* data;
  int64_t size[4];
  int64_t stride[4];
} omm_view4;

/* Top-k visibility rule (reference cuda_backend/csrc/topk.cu:15-97), in tokens:
 *   query row g covers tokens [g*group_size, ...); q_cid = (g*group_size)/chunk_q + q_chunk_offset
 *   key block c: k_cid = blocks_per_chunk > 0 ? c / blocks_per_chunk
 *                                             : (c*block_size) / chunk_k
 * With group_size | chunk_q and blocks_per_chunk == 0 this is the reference's rule with
 * chunk_size = chunk_q / group_size and chunk_size_k = chunk_k.  blocks_per_chunk > 0 is the
 * chunk-aligned page layout of the paged cache (a chunk's last page may be partial). */
typedef struct omm_topk_mask {
  int32_t block_size;
  int32_t group_size;
  int32_t chunk_q;
  int32_t chunk_k;
  int32_t blocks_per_chunk;
  int32_t q_chunk_offset;
  int32_t q_half;   /* tf_mask only: clean query chunks */
  int32_t k_half;   /* tf_mask only: clean key chunks */
  int32_t ex_win;
  int32_t ex_sink;
  int32_t causal;
  int32_t tf_mask;
  int32_t prog_excl;
} omm_topk_mask;

/* Paged block KV cache of one layer.  A unit is one (head, chunk): pages_per_chunk pages of
 * page_tokens tokens x head_dim, stored contiguously at slot s of pool_k / pool_v.  Units not
 * resident in HBM live in a pinned host pool (zero-copy readable by the device). */
typedef struct omm_paged_kv {
  void* pool_k;               /* [n_slots][pages_per_chunk][page_tokens][head_dim] */
  void* pool_v;
  float* scale_k;             /* fp8 only: [n_slots][pages_per_chunk] dequant scales */
  float* scale_v;
  const void* host_k;         /* device-visible pinned host pool, same unit layout */
  const void* host_v;
  const float* host_scale_k;
  const float* host_scale_v;
  const int32_t* unit_table;  /* [num_heads][max_chunks]: s >= 0 HBM slot; s <= -2 host slot
                                 (-2 - s); -1 never written */
  int32_t num_heads;
  int32_t max_chunks;
  int32_t n_chunks;           /* chunks 0 .. n_chunks-1 are readable */
  int32_t chunk_len;          /* tokens per chunk (4680 for 3 Wan latent frames) */
  int32_t page_tokens;        /* 64 */
  int32_t pages_per_chunk;    /* ceil(chunk_len / page_tokens) */
  int32_t head_dim;           /* 128 */
  int32_t dtype;              /* OMM_BF16 or OMM_FP8E4M3 */
  int32_t n_slots;            /* HBM unit slots */
  int32_t n_host_slots;
} omm_paged_kv;

/* ---- library ------------------------------------------------------------------------- */
const char* omm_last_error(void);
int omm_abi_version(void); /* 1 */

/* Pinned, device-mapped host memory for the cache's host pool; *dev receives the device
 * address (equal to *host on ROCm with unified addressing, but always use *dev on device). */
int omm_host_alloc(size_t bytes, void** host, void** dev);
int omm_host_free(void* host);

/* ---- block compression / query pooling (a1, a2) -------------------------------------- */
/* out[b, j, h, :] = mean over tokens t in [j*group, min((j+1)*group, T)) of x[b, t, h, :].
 * fp32 accumulation in ascending token order, one IEEE division by the token count, one
 * round-to-nearest-even to the element type.  x: [B, T, H, D]; out: [B, ceil(T/group), H, D]. */
int omm_block_pool(const omm_view4* x, const omm_view4* out, int32_t dtype, int32_t group,
                   void* stream);

/* ---- block scoring + top-k (a3, a4) -------------------------------------------------- */
size_t omm_topk_workspace_bytes(int64_t B, int64_t MG, int64_t H, int64_t NC, int32_t topk);
/* q: pooled queries [B, MG, H, D]; k: compressed keys [B, NC, H, D]; out: int32 contiguous
 * [B, MG, H, topk].  score = (sum_d fmaf(q_d, k_d, acc), d ascending) * scale in fp32.
 * Valid slots hold block ids in (score desc, id asc) order (+0 == -0); -1 pads rows with fewer
 * than topk visible blocks.  Invisible blocks and scores that are -inf or NaN are never
 * selected.  1 <= topk <= 64, D <= 256. */
int omm_topk(const omm_view4* q, const omm_view4* k, int32_t dtype, int32_t topk, float scale,
             const omm_topk_mask* mask, int32_t* out, void* workspace, size_t workspace_bytes,
             void* stream);
/* q: full-resolution queries [B, T, H, D]; row g pools tokens [g*group_size,
 * min((g+1)*group_size, T)) exactly as omm_block_pool (fp32 sum in ascending token order, one
 * division, one rounding to the element type), then scores and selects as omm_topk.  Rows are
 * pooled inside the top-k kernel when the shape allows (q read once); otherwise into the
 * workspace first.  out: int32 contiguous [B, ceil(T/group_size), H, topk]. */
size_t omm_topk_fused_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int64_t NC,
                                      int32_t group_size, int32_t topk, int32_t dtype);
int omm_topk_fused(const omm_view4* q, const omm_view4* k, int32_t dtype, int32_t group_size,
                   int32_t topk, float scale, const omm_topk_mask* mask, int32_t* out,
                   void* workspace, size_t workspace_bytes, void* stream);
/* scores: fp32 contiguous [B, MG, H, NC], already scaled; same selection and output as above. */
int omm_topk_from_scores(const float* scores, int64_t B, int64_t MG, int64_t H, int64_t NC,
                         int32_t topk, const omm_topk_mask* mask, int32_t* out, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ---- selection attention forward, dense K/V (a5) ------------------------------------- */
/* q: [B, M, H, D]; k, v: [B, N, H, D]; ids: int32 [B, MG, H, T], MG = ceil(M / group_size);
 * out: [B, M, H, D] (q dtype); lse: fp32 contiguous [B, H, M] or NULL.
 * Query m (group g = m / group_size) attends to the tokens of its listed blocks (0 <= id,
 * id*block_size < N; causal: (id*block_size)/chunk_size <= q_chunk and token/chunk_size <=
 * q_chunk with q_chunk = (g*group_size)/chunk_size).  No visible token: out 0, lse -inf.
 * bf16/f16 run on MFMA with bf16/f16 P; f32 runs full fp32 arithmetic. */
int omm_sel_fwd(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                const omm_view4* ids, int32_t dtype, int32_t block_size, int32_t chunk_size,
                int32_t causal, int32_t group_size, float scale, const omm_view4* out,
                float* lse, void* stream);

/* ---- pointer-table selection (a6, reference address contract) ------------------------ */
/* bf16 only.  ptr tables: int64 [B, MG, H, T] with element strides ptr_stride; a block is
 * block_size full rows at (address + r*stride_bn + d*stride_bd) elements; 0 = skip. */
int omm_sel_fwd_ptr(const omm_view4* q, const int64_t* ptr_k, const int64_t* ptr_v,
                    const int64_t* ptr_stride, int64_t T, int32_t block_size, int32_t group_size,
                    int64_t stride_bn, int64_t stride_bd, float scale, const omm_view4* out,
                    float* lse, void* stream);

/* ---- paged block KV cache (a7) ------------------------------------------------------- */
/* Selection attention over the cache, non-causal.  q: bf16 [1, M, H, D]; ids: int32
 * [1, MG, H, T] of chunk-aligned page ids (page p of chunk c is id c*pages_per_chunk + p,
 * with min(page_tokens, chunk_len - p*page_tokens) valid tokens). */
int omm_sel_fwd_paged(const omm_view4* q, const omm_view4* ids, const omm_paged_kv* kv,
                      int32_t group_size, float scale, const omm_view4* out, float* lse,
                      void* stream);

#ifdef __cplusplus
}
#endif
#endif /* OMNIMEM_HIP_H_ */
