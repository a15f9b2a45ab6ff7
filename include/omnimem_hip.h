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
 *   omm_sel_fwd_ws          <- the same op with a workspace for the split fp32 path (the
 *                              reference's fp32 kernel takes none: selection_fwd.cu:820-932)
 *   omm_sel_bwd             <- torch.ops.omnimem_nsa.sel_bwd (bindings.cpp:25-28, ops.h:38-43,
 *                              selection_bwd.cu:1329-1407) with its inverted index
 *                              (inverted_index.cu:103-177)
 *   omm_sel_fwd_ptr         <- torch.ops.omnimem_nsa.sel_fwd_ptr (bindings.cpp:20-23,
 *                              selection_fwd.cu:968-992)
 *   omm_build_ptr_table     <- torch.ops.omnimem_nsa.build_ptr_table (bindings.cpp:12-15,
 *                              ptr_table.cu:59-127)
 *   omm_sel_bwd_ptr         <- torch.ops.omnimem_nsa.sel_bwd_ptr (bindings.cpp:29-35,
 *                              selection_bwd.cu:1409-1529; Triton twin
 *                              padded_ptr/kernels/select_bwd.py:564-711)
 *   omm_paged_append        <- MMCache.update_cache chunk_per_head branch (models/cache.py:478-502)
 *                              fused with the K / V block compression
 *                              (causal_wan_nsa_model.py:479-490)
 *   omm_paged_append_ring   <- the same, also writing the chunk into a bf16 window ring slot
 *   omm_copy_units          <- flush_offload D2H (models/cache.py:1086-1117) and the reload H2D
 *                              (nsa/ops/selection/padded_ptr/wrapper.py:342-361)
 *   omm_gather_publish_clear, omm_block_range, omm_dedup_run
 *                           <- block-KV K1 / K2 / K3 (cuda_backend/csrc/block_kv_ops.h:12-31)
 *   omm_sel_fwd_paged       <- selection_attention_padded_ptr_fast
 *                              (nsa/ops/selection/padded_ptr/wrapper.py:458-553) over the paged
 *                              cache, with int32 unit slots instead of raw int64 addresses
 *   omm_sel_fwd_paged_gated <- the same, with the branch mix of causal_wan_nsa_model.py:541-546
 *   omm_sel_fwd_gated       <- sel_fwd with that branch mix, for the full-sequence branch
 *                              (causal_wan_nsa_model.py:391-458, 541-546)
 *   omm_paged_stage         <- the reload of missing blocks before a selection
 *                              (padded_ptr/wrapper.py:268-361), per page on a side stream
 *   omm_copy_units_async    <- flush_offload's D2H copies (models/cache.py:1086-1117) on the
 *                              copy engines
 *   omm_host_alloc / _free  <- MMCache's pinned offload buffers (models/cache.py:970-1016)
 *   omm_topk_fused_noalloc, omm_topk_fused_debug: no reference counterpart (callers that cannot
 *                              allocate; a test hook that also returns the scores)
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
 * resident in HBM live in a pinned host pool that the device reads directly.  The pools may be
 * shared by all layers (slots are global); unit_table and stamp are per layer. */
typedef struct omm_paged_kv {
  void* pool_k;               /* [n_slots][pages_per_chunk][page_tokens][head_dim] */
  void* pool_v;
  float* scale_k;             /* fp8 only: [n_slots][pages_per_chunk] dequantisation scales */
  float* scale_v;
  void* host_k;               /* device address of the pinned host pool, same unit layout */
  void* host_v;
  float* host_scale_k;        /* fp8 only: [n_host_slots][pages_per_chunk] */
  float* host_scale_v;
  const int32_t* unit_table;  /* [num_heads][max_chunks]: s >= 0 HBM slot; s <= -2 host slot
                                 (-2 - s); -1 never written */
  int32_t* stamp;             /* [num_heads][max_chunks] epoch of the last touch, or NULL */
  int32_t* reads;             /* [num_heads][max_chunks] pages read since the caller last
                                 cleared it (residency policy input), or NULL */
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
  uint8_t* page_seen;         /* [num_heads][max_chunks][pages_per_chunk]: set to 1 for every
                                 page a selection lists since the caller last cleared it (unique
                                 pages read, e.g. host-link bytes), or NULL */
  int32_t qk_fp8;             /* fp8 caches: 1 = quantise the queries to e4m3 per query row
                                 (scale amax / 448) and compute Q K^T on fp8 MFMA with the K page
                                 codes (head dim 64 / 128); 0 = K codes widened to bf16
                                 (bf16 MFMA; the page scales apply to the scores) */
  int32_t* touches;           /* [num_heads][max_chunks]: += 1 the first time a selection call
                                 (one epoch) reads the unit, i.e. the reference's per-call LRU
                                 accesses (models/cache.py:673-699), or NULL; needs kv->stamp */
  /* HBM staging of host-resident pages (omm_paged_stage), or stage_map_epoch == NULL: */
  void* stage_k;              /* [stage_slots][page_tokens][head_dim] pages, cache dtype */
  void* stage_v;
  float* stage_scale_k;       /* fp8 only: [stage_slots] */
  float* stage_scale_v;
  int32_t* stage_map_epoch;   /* [num_heads][max_chunks][pages_per_chunk]: epoch of the call
                                 that staged the page last */
  int32_t* stage_map_slot;    /* same shape: its staging slot, or -1 (pool full: read in place) */
  int32_t* stage_counter;     /* 1 int32: slots taken by the current call */
  int32_t stage_slots;
} omm_paged_kv;

/* ---- library ------------------------------------------------------------------------- */
const char* omm_last_error(void);
int omm_abi_version(void); /* 4 */

/* Pinned, device-mapped host memory for the cache's host pool; *dev receives the device
 * address (equal to *host on ROCm with unified addressing, but always use *dev on device).
 * Reference: the pinned offload buffers of MMCache.preallocate_offload_buffer
 * (models/cache.py:970-1016) and the pinned tensors of its eviction path (cache.py:853,906). */
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
 * [B, MG, H, topk].  Scores are fp32, scale * <q, k>, computed one of two ways:
 *  - MFMA path: bf16 / f16 inputs, head dim 64 or 128, topk <= 16, unit dim strides and 16-byte
 *    aligned rows.  The products are exact and the fp32 sum runs in the matrix cores' order, so
 *    a score lies within the fp32 summation bound of the exact dot product (not bit-equal to
 *    the fmaf chain below); the selection is exact on these scores.
 *  - VALU path (every other input, fp32 included): score = (sum_d fmaf(q_d, k_d, acc),
 *    d ascending) * scale, bit-reproducible by a scalar fmaf loop.
 * For topk <= 128 (the reference's path A, topk.cu:584, 648-660) valid slots hold block ids in
 * (score desc, id asc) order (+0 == -0); -1 pads rows with fewer than topk visible blocks;
 * invisible blocks and scores that are -inf or NaN are never selected.  For 128 < topk <= 4096
 * the reference's path B rule applies (topk.cu:741-807): each visible block is ranked by the
 * raw order code of its score (+0 above -0; -inf and NaN ranked too, a NaN with the sign bit
 * clear first), hidden blocks come last as -1, ties by id ascending, -1 past NC.  That path
 * writes every row's scores to the workspace (omm_topk_workspace_bytes) and selects per row.
 * D <= 256.  An empty output (B, MG or H zero) launches nothing and out may be NULL; NC = 0
 * fills out with -1. */
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
/* Test hook, no reference counterpart: omm_topk_fused that also writes the fp32 scores its
 * selection ran on into scores ([B, ceil(T/group_size), H, NC], contiguous; entries of columns
 * a row cannot see may be left unwritten), so the selection can be checked bit for bit against
 * the reference rule on identical scores.  MFMA path only (bf16 / f16, head dim 64 or 128,
 * unit dim strides, 16-byte aligned rows); other inputs fail with OMM_EUNSUPPORTED. */
int omm_topk_fused_debug(const omm_view4* q, const omm_view4* k, int32_t dtype,
                         int32_t group_size, int32_t topk, float scale,
                         const omm_topk_mask* mask, int32_t* out, float* scores,
                         void* workspace, size_t workspace_bytes, void* stream);
/* No counterpart in the reference: omm_topk_fused for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).  Same arguments
 * and result as omm_topk_fused without the workspace: the workspace is a fixed array of
 * omm_topk_fused_noalloc_max_bytes() bytes in the library's device memory, one per GPU, held
 * until the process ends.  A call whose omm_topk_fused_workspace_bytes exceeds that size fails
 * with OMM_EWORKSPACE.  Calls that overlap on one GPU (two streams, or two threads) race on the
 * array; serialise them.  Nothing in the array needs to start at zero. */
size_t omm_topk_fused_noalloc_max_bytes(void);
int omm_topk_fused_noalloc(const omm_view4* q, const omm_view4* k, int32_t dtype,
                           int32_t group_size, int32_t topk, float scale,
                           const omm_topk_mask* mask, int32_t* out, void* stream);
/* scores: fp32 contiguous [B, MG, H, NC], already scaled; same selection and output as above
 * (topk > 128 needs no workspace here). */
int omm_topk_from_scores(const float* scores, int64_t B, int64_t MG, int64_t H, int64_t NC,
                         int32_t topk, const omm_topk_mask* mask, int32_t* out, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ---- selection attention forward, dense K/V (a5) ------------------------------------- */
/* q: [B, M, H, D]; k, v: [B, N, H, D]; ids: int32 [B, MG, H, T], MG = ceil(M / group_size);
 * out: [B, M, H, D] (q dtype); lse: fp32 contiguous [B, H, M] or NULL.
 * Query m (group g = m / group_size) attends to the tokens of its listed blocks (0 <= id,
 * id*block_size < N; causal: (id*block_size)/chunk_size <= q_chunk and token/chunk_size <=
 * q_chunk with q_chunk = (g*group_size)/chunk_size).  No visible token: out 0, lse -inf.
 * bf16/f16 run on MFMA with bf16/f16 P; f32 runs full fp32 arithmetic.  Offsets are 32-bit
 * where they can be: ids must span fewer than 2^31 elements and each (b, h) slice of k / v
 * fewer than 2^32 (OMM_EUNSUPPORTED otherwise). */
int omm_sel_fwd(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                const omm_view4* ids, int32_t dtype, int32_t block_size, int32_t chunk_size,
                int32_t causal, int32_t group_size, float scale, const omm_view4* out,
                float* lse, void* stream);
/* omm_sel_fwd with a device workspace (same reference op; the workspace is this library's own).
 * An f32 call with few (b, query group, head) items for the current device's CUs splits its
 * selected blocks into equal runs, one per workgroup, and merges the split items' partial
 * results in a second pass through the workspace: all CUs get the same work (config 1:
 * 300 items on 256 CUs).  omm_sel_fwd_workspace_bytes gives the size for a call (ids [B, MG, H,
 * T]); 0 means no split, and so does a NULL or smaller workspace: then the call is
 * omm_sel_fwd.  The workspace is 16-byte aligned, must not overlap the other arguments, and is
 * in use until the call's work on the stream ends; nothing in it needs to start at zero.
 * Results agree with omm_sel_fwd's within fp32 rounding (the sums run in another order). */
size_t omm_sel_fwd_workspace_bytes(int64_t B, int64_t M, int64_t H, int64_t D, int64_t T,
                                   int32_t dtype, int32_t group_size);
int omm_sel_fwd_ws(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                   const omm_view4* ids, int32_t dtype, int32_t block_size, int32_t chunk_size,
                   int32_t causal, int32_t group_size, float scale, const omm_view4* out,
                   float* lse, void* workspace, size_t workspace_bytes, void* stream);
/* The same selection (bf16 only) with the NSA branch mix of causal_wan_nsa_model.py:541-546 in
 * its epilogue, for the full-sequence branch (:391-458):
 *   out = g[..., 0] * o_cmp + g[..., 1] * o_slc + g[..., 2] * o_swa
 * in fp32 from the unrounded o_slc, one rounding to bf16.  gates: bf16 [B, M, H, 3] (after the
 * clamp and sigmoid); o_cmp, o_swa: bf16 of q's shape, unit dim stride, 16-byte aligned rows;
 * out must not overlap them.  lse stays that of the selection alone.  Needs the MFMA path (head
 * dim 64 or 128, 16-byte q / out rows, a finite non-zero scale), else OMM_EUNSUPPORTED. */
int omm_sel_fwd_gated(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                      const omm_view4* ids, int32_t block_size, int32_t chunk_size,
                      int32_t causal, int32_t group_size, float scale, const omm_view4* gates,
                      const omm_view4* o_cmp, const omm_view4* o_swa, const omm_view4* out,
                      float* lse, void* stream);
/* ---- selection attention backward, dense K/V -------------------------------------------- */
/* Reference: torch.ops.omnimem_nsa.sel_bwd (bindings.cpp:25-28, ops.h:38-43,
 * selection_bwd.cu:1329-1407) and the inverted index it builds (inverted_index.cu:103-177).
 * Same arguments as omm_sel_fwd plus the forward's out and lse (fp32 contiguous [B, H, M]) and
 * d_out ([B, M, H, D], q dtype).  With delta_m = sum_d out[m,d] d_out[m,d] (fp32),
 * P = exp(q.k * scale - lse) (0 for rows with lse = -inf) and dS = P (d_out.v - delta) scale:
 * dq = dS K (q dtype), dk = dS^T Q and dv = P^T d_out over every (query, token) pair the forward
 * attends to (k dtype, fp32 accumulation, one rounding).  Every element of dq, dk and dv is
 * written (0 for tokens no query sees).  Duplicated ids in a row count twice, as in the
 * forward.  bf16 / f16 with head dim 64 or 128, unit dim strides and 16-byte aligned rows run on
 * MFMA (16-bit P and dS operands); f32 and every other head dim <= 256 or stride run full fp32
 * arithmetic.  The workspace (256-byte aligned) holds delta, -lse log2 e, the per-block CSR
 * offsets and the bucket lists. */
size_t omm_sel_bwd_workspace_bytes(int64_t B, int64_t M, int64_t H, int64_t N,
                                   int32_t block_size, int32_t group_size, int64_t T);
int omm_sel_bwd(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                const omm_view4* ids, const omm_view4* out, const float* lse,
                const omm_view4* d_out, int32_t dtype, int32_t block_size, int32_t chunk_size,
                int32_t causal, int32_t group_size, float scale, const omm_view4* dq,
                const omm_view4* dk, const omm_view4* dv, void* workspace,
                size_t workspace_bytes, void* stream);

/* ---- pointer-table selection (a6, reference address contract) ------------------------ */
/* ptr_x[b,g,h,t] = base_x[h, cid] + b*batch_stride + (bid % bpc)*in_chunk_block_bytes with
 * cid = bid / bpc (bpc > 0) or bid (bpc == 0); 0 when bid < 0, bid >= n_blocks_per_head[h],
 * cid >= max_chunks or base == 0.  ids: int32 [B, MG, H, T]; base_x: int64 byte addresses with
 * element strides base_stride_h / base_stride_c; ptr_k / ptr_v: int64 contiguous [B, MG, H, T]. */
int omm_build_ptr_table(const omm_view4* ids, const int64_t* base_k, const int64_t* base_v,
                        int64_t base_stride_h, int64_t base_stride_c, int32_t max_chunks,
                        const int32_t* n_blocks_per_head, int64_t batch_stride,
                        int32_t blocks_per_chunk, int64_t in_chunk_block_bytes, int64_t* ptr_k,
                        int64_t* ptr_v, void* stream);
/* bf16 only.  ptr tables: int64 [B, MG, H, T] with element strides ptr_stride; a block is
 * block_size full rows at (address + r*stride_bn + d*stride_bd) elements; 0 = skip.  Any
 * 2-byte-aligned address is accepted: blocks that are not 16-byte aligned are detected per
 * block on the device and read with 2-byte loads (slower, same result). */
int omm_sel_fwd_ptr(const omm_view4* q, const int64_t* ptr_k, const int64_t* ptr_v,
                    const int64_t* ptr_stride, int64_t T, int32_t block_size, int32_t group_size,
                    int64_t stride_bn, int64_t stride_bd, float scale, const omm_view4* out,
                    float* lse, void* stream);
/* Pointer-table backward (the padded-pointer training path).  q, out, d_out, dq: bf16
 * [B, M, H, D]; lse: the forward's fp32 contiguous [B, H, M]; ids: int32 [B, MG, H, T]; ptr_k /
 * ptr_v: the forward's address tables (element strides ptr_stride[4]).  Writes dq (q dtype) and
 * delta (fp32 contiguous [B, H, M], delta_m = sum_d out[m,d] d_out[m,d]).
 * dQ: P = exp(q.k * scale - lse) over the block_size rows of every nonzero (ptr_k, ptr_v) slot
 * (0 for rows with lse = -inf), dS = P (d_out.v - delta) scale, dq = dS K.
 * With compute_dkv: block id bid of head h resolves, as omm_build_ptr_table does, through the
 * [H, max_base] base tables (element strides base_stride[0], base_stride[1]) to K / V at
 * base_k/v[h, bid / bpc] + b*batch_stride_kv_bytes + (bid % bpc)*in_chunk_block_bytes_kv (bpc =
 * blocks_per_chunk > 0; else base[h, bid]) and to fp32 dK / dV scratch at base_dk/dv[...] +
 * b*batch_stride_dkv_bytes + (bid % bpc)*in_chunk_block_bytes_dkv, rows stride_dbn / dims
 * stride_dbd elements.  It is skipped (nothing read or written) when bid >= n_blocks_per_head[h]
 * (if given), bid / bpc >= max_base or any of its four bases is 0.  Every resolved block of
 * bid < max_base*bpc (max_base when bpc == 0) gets dK = sum dS^T Q and dV = sum P^T d_out over the
 * (group, slot) pairs that list it with 0 <= id < n_blocks_per_head[h] (all block_size rows
 * written; 0 when none does; stored, not added).  Duplicated ids count twice.  MFMA kernels for
 * head dim 64 / 128 with stride_bd == 1 and stride_bn % 8 == 0 (block addresses may be 2-byte
 * aligned), VALU fp32 kernels otherwise (head dim <= 256).  Workspace (256-byte aligned): -lse
 * log2 e and, with compute_dkv, the per-block CSR offsets and bucket lists. */
size_t omm_sel_bwd_ptr_workspace_bytes(int64_t B, int64_t M, int64_t H, int64_t max_base,
                                       int32_t blocks_per_chunk, int32_t group_size, int64_t T,
                                       int32_t compute_dkv);
int omm_sel_bwd_ptr(const omm_view4* q, const omm_view4* out, const float* lse,
                    const omm_view4* d_out, const omm_view4* ids, const int64_t* ptr_k,
                    const int64_t* ptr_v, const int64_t* ptr_stride, const int64_t* base_k,
                    const int64_t* base_v, const int64_t* base_dk, const int64_t* base_dv,
                    const int64_t* base_stride, int64_t max_base,
                    const int32_t* n_blocks_per_head, int32_t block_size, int32_t group_size,
                    int64_t batch_stride_kv_bytes, int64_t batch_stride_dkv_bytes,
                    int64_t stride_bn, int64_t stride_bd, int64_t stride_dbn, int64_t stride_dbd,
                    int32_t blocks_per_chunk, int64_t in_chunk_block_bytes_kv,
                    int64_t in_chunk_block_bytes_dkv, float scale, int32_t compute_dkv,
                    const omm_view4* dq, float* delta, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ---- paged block KV cache (a7) ------------------------------------------------------- */
/* Write chunk cid of every head from k_new / v_new (bf16 [1, chunk_tokens, H, D], unit dim
 * stride, 16-byte aligned rows; chunk_tokens == chunk_len: whole chunks only, so every page
 * slot attention reads was written) into the units unit_table[h][cid] (HBM slots; units whose
 * entry is < 0 are skipped).  The last page's slots past chunk_len are zeroed.
 * bf16 cache: bytes copied.  fp8 cache: per (page, head) scale = amax/448 (1 when amax == 0),
 * code = e4m3(clamp(x * (448/amax), +-448)), round to nearest even.  With k_cmp (bf16
 * [1, >= (cid+1)*pages_per_chunk, H, D]) row cid*pages_per_chunk + p receives the mean of page
 * p's keys (omm_block_pool arithmetic over its valid tokens; 0 for a page with none), and
 * v_cmp the same for the values (both optional).  With kv->stamp and epoch > 0,
 * stamp[h][cid] = epoch.
 * Reference: MMCache.update_cache, chunk_per_head branch (models/cache.py:478-502) and the K
 * block compression of causal_wan_nsa_model.py:479-484. */
int omm_paged_append(const omm_paged_kv* kv, const omm_view4* k_new, const omm_view4* v_new,
                     int32_t cid, int32_t chunk_tokens, const omm_view4* k_cmp,
                     const omm_view4* v_cmp, int32_t epoch, void* stream);
/* omm_paged_append that also copies k_new / v_new bit for bit into ring_k / ring_v (bf16
 * [1, chunk_tokens, H, D], unit dim stride, 16-byte aligned rows, apart from k_new / v_new; each
 * optional): the slot of a bf16 window ring that an fp8 cache keeps for the window branch
 * (MMCache.update_cache also returns the window K/V it stores, models/cache.py:478-502,
 * 576-588).  With head dim 64 / 128 and pages of <= 64 tokens the append kernel writes the
 * copies from its registers, so the chunk is read once. */
int omm_paged_append_ring(const omm_paged_kv* kv, const omm_view4* k_new,
                          const omm_view4* v_new, int32_t cid, int32_t chunk_tokens,
                          const omm_view4* k_cmp, const omm_view4* v_cmp, const omm_view4* ring_k,
                          const omm_view4* ring_v, int32_t epoch, void* stream);
/* Selection attention over the cache, non-causal.  q: bf16 [1, M, H, D]; ids: int32
 * [1, MG, H, T] (spanning fewer than 2^31 elements) of chunk-aligned page ids (page p of chunk c is id c*pages_per_chunk + p,
 * with min(page_tokens, chunk_len - p*page_tokens) valid tokens); ids outside the readable
 * chunks or of units never written are skipped.  With kv->stamp and epoch > 0 every unit read
 * gets stamp = epoch (the LRU touch of the reference's _touch_lru_and_detect_missing,
 * nsa/ops/selection/padded_ptr/wrapper.py:253-291, without its host synchronisation); with
 * kv->reads, reads[h][cid] += 1 for every listed page of the unit; with kv->touches as well,
 * touches[h][cid] += 1 once per call (the unit's stamp moving to this epoch counts it). */
int omm_sel_fwd_paged(const omm_view4* q, const omm_view4* ids, const omm_paged_kv* kv,
                      int32_t group_size, float scale, const omm_view4* out, float* lse,
                      int32_t epoch, void* stream);
/* Stage the host-resident pages that a selection call with these ids will read: each distinct
 * (head, chunk, page) of a host-pool unit listed in ids is copied once into the staging pool
 * (K, V and, for fp8, the page scales), and stage_map_epoch / stage_map_slot record where, under
 * `epoch`.  A later omm_sel_fwd_paged / _gated call with the same epoch and kv reads those pages
 * from the pool (bit-identical bytes) instead of over the host link page by page; pages that
 * did not fit (more than stage_slots) are read in place as before.  Enqueue it on a side stream
 * right after the top-k, ordered before the selection by an event, and the copies overlap the
 * work in between.  One call in flight per staging pool; epochs must be unique per call.
 * Reference: the block store's prepare_selection (nsa/ops/selection/padded_ptr/
 * block_wrapper.py:51-85) over K3 dedup (csrc/block_kv_dedup.cu:134-206) and K1 gather
 * (csrc/block_kv_gather.cu:14-45), whose per-call gather of missing blocks into a pool this
 * replaces for the paged cache. */
int omm_paged_stage(const omm_paged_kv* kv, const omm_view4* ids, int32_t epoch, void* stream);
/* The same selection with the NSA branch mix fused into its epilogue:
 *   out = g[..., 0] * o_cmp + g[..., 1] * o_slc + g[..., 2] * o_swa
 * per (query, head), in fp32 with one rounding to bf16, where o_slc is the selection output
 * and lse, when given, is the selection's.  bf16 caches fuse the mix into the selection kernel's
 * epilogue (o_slc is never written separately); fp8 caches write o_slc (rounded to bf16) and mix
 * it in a second pass over out.  gates: bf16 [1, M, H, 3] (the branch gates after their
 * sigmoid), o_cmp / o_swa: bf16 [1, M, H, D] with unit dim stride and 16-byte aligned rows.
 * Needs the MFMA path (head dim 64 or 128, 16-byte q / out rows, finite non-zero scale).
 * Aliasing: on a bf16 cache out may be the very view o_cmp or o_swa is (same address and
 * strides: each element is read before it is written, by the same thread); any other overlap of
 * out with o_cmp or o_swa, and on an fp8 cache any overlap at all (its first pass writes out
 * before the mix reads the branches), is rejected with OMM_EINVAL.
 * Reference: the gate combine of causal_wan_nsa_model.py:541-546 after the three branches. */
int omm_sel_fwd_paged_gated(const omm_view4* q, const omm_view4* ids, const omm_paged_kv* kv,
                            int32_t group_size, float scale, const omm_view4* gates,
                            const omm_view4* o_cmp, const omm_view4* o_swa, const omm_view4* out,
                            float* lse, int32_t epoch, void* stream);
/* Batched unit copies: for i < n copy unit_bytes from src_k + src_slot[i]*unit_bytes to
 * dst_k + dst_slot[i]*unit_bytes (either side may be the mapped host pool), the same for the
 * optional V pair and the optional scale pairs (scale_bytes per unit).  src_slot / dst_slot are
 * device int32 arrays; entries outside [0, n_src_slots) / [0, n_dst_slots) are skipped.  Reference: flush_offload's D2H copies (models/cache.py:1086-1117) and
 * the reload H2D of wrapper.py:342-361, as one launch. */
int omm_copy_units(const void* src_k, void* dst_k, const void* src_v, void* dst_v,
                   const void* src_sk, void* dst_sk, const void* src_sv, void* dst_sv,
                   const int32_t* src_slot, const int32_t* dst_slot, int32_t n,
                   int32_t n_src_slots, int32_t n_dst_slots, int64_t unit_bytes,
                   int64_t scale_bytes, void* stream);
/* The same moves with the slot lists in host memory, each unit (K, V and, when given, the two
 * scale arrays) one hipMemcpyAsync on `stream`: the copy engines move the bytes, no kernel runs,
 * so a side stream's moves do not occupy compute units beside the attention kernels.  Runs of
 * units consecutive in both pools are merged into one copy.  Reference: the same flush_offload
 * D2H (models/cache.py:1086-1117), whose pinned-buffer copies are non_blocking. */
int omm_copy_units_async(const void* src_k, void* dst_k, const void* src_v, void* dst_v,
                         const void* src_sk, void* dst_sk, const void* src_sv, void* dst_sv,
                         const int32_t* src_slot_host, const int32_t* dst_slot_host, int32_t n,
                         int32_t n_src_slots, int32_t n_dst_slots, int64_t unit_bytes,
                         int64_t scale_bytes, void* stream);

/* ---- reference block-store kernels (K1 / K2 / K3) ------------------------------------ */
/* K1 (cuda_backend/csrc/block_kv_ops.h:12-16, block_kv_gather.cu:14-45): desc is int64
 * [6*n_fetch + n_clear], SoA [src_k|src_v|dst_k|dst_v|pub_k|pub_v] x n_fetch then the clear
 * addresses.  Copies block_bytes from src to dst (K and V), then stores dst into *pub; zeroes
 * the int64 at each clear address.  *ctas receives the workgroups launched. */
int omm_gather_publish_clear(const int64_t* desc, int64_t n_fetch, int64_t n_clear,
                             int64_t block_bytes, int64_t* ctas, void* stream);
/* K2 (block_kv_ops.h:18-23, block_kv_range.cu:13-37): table int64 contiguous [2, heads, mb];
 * table[x][h][first_bid + j] = base_x + h*head_stride_bytes + j*block_bytes (0 when clear) for
 * j < n_blocks; n_valid[h] = n_valid_value when >= 0. */
int omm_block_range(int64_t* table, int32_t* n_valid, int64_t heads, int64_t mb,
                    int64_t first_bid, int64_t n_blocks, int64_t k_base, int64_t v_base,
                    int64_t head_stride_bytes, int64_t block_bytes, int64_t n_valid_value,
                    int32_t write_k, int32_t write_v, int32_t clear, void* stream);
/* K3 (block_kv_ops.h:25-31, block_kv_dedup.cu:16-206): entry e of the flattened [B, MG, H, t]
 * block_indices with 0 <= bid < mb is head h = (e / t) % heads and key (cid*heads + h)*bpc +
 * loc for bid = cid*bpc + loc.  out[0] = number of distinct keys, out[1..] the distinct keys
 * ascending (at most cap written).  stamp: int32 [heads*mb], persistent between calls (epochs
 * must differ); counts / offsets: int32 [>= ceil(heads*mb / 1024)]. */
int omm_dedup_run(const int32_t* block_indices, int64_t n_entries, int32_t* stamp,
                  int32_t* counts, int32_t* offsets, int32_t* out, int64_t epoch, int64_t mb,
                  int64_t heads, int64_t t, int64_t bpc, int64_t cap, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* OMNIMEM_HIP_H_ */
