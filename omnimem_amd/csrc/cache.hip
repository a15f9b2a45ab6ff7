// Block KV cache kernels: the paged cache (append with fused block compression and fp8
// quantisation, batched unit copies for evict / promote), the reference's pointer-table builder,
// and the reference's block-store kernels K1 (gather + publish + clear), K2 (table range) and
// K3 (dedup of selected blocks).
//
// Reference semantics: cuda_backend/csrc/ptr_table.cu:1-55 (address contract, 0 = skip),
// block_kv_ops.h:1-31 (K1/K2/K3 contracts), models/cache.py:478-502 (per-head chunk append).
// Paged layout (new): a unit is one (head, chunk) of one layer, pages_per_chunk pages of
// page_tokens x head_dim elements, contiguous; units live in HBM slots or in a device-mapped
// pinned host pool and are addressed through an int32 unit table instead of raw addresses.
#include "omm_common.h"

namespace omm {
namespace {

// ---- pointer table (reference address contract) ------------------------------------------------
__global__ __launch_bounds__(256) void ptr_table_kernel(
    const int32_t* __restrict__ ids, int64_t is0, int64_t is1, int64_t is2, int64_t is3,
    const int64_t* __restrict__ base_k, const int64_t* __restrict__ base_v, int64_t bsh,
    int64_t bsc, int max_chunks, const int32_t* __restrict__ n_blocks, int64_t* __restrict__ pk,
    int64_t* __restrict__ pv, int MG, int H, int T, int64_t batch_stride, int bpc,
    int64_t in_chunk_bytes, int64_t total) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int t = static_cast<int>(i % T);
    const int64_t r1 = i / T;
    const int h = static_cast<int>(r1 % H);
    const int64_t r2 = r1 / H;
    const int g = static_cast<int>(r2 % MG);
    const int b = static_cast<int>(r2 / MG);
    const int32_t bid = ids[b * is0 + g * is1 + h * is2 + t * is3];
    int64_t ak = 0, av = 0;
    if (bid >= 0 && bid < n_blocks[h]) {
      const int64_t cid = bpc > 0 ? bid / bpc : bid;
      const int64_t off = bpc > 0 ? static_cast<int64_t>(bid % bpc) * in_chunk_bytes : 0;
      if (cid < max_chunks) {
        const int64_t bk = base_k[h * bsh + cid * bsc], bv = base_v[h * bsh + cid * bsc];
        const int64_t delta = static_cast<int64_t>(b) * batch_stride + off;
        ak = bk != 0 ? bk + delta : 0;
        av = bv != 0 ? bv + delta : 0;
      }
    }
    pk[i] = ak;
    pv[i] = av;
  }
}

// ---- paged append ----------------------------------------------------------------------------
struct AppendArgs {
  const bf16_t* k;     // new chunk [1, S, H, D] (token stride ks1, head stride ks2)
  const bf16_t* v;
  int64_t ks1, ks2, vs1, vs2;
  void* pool_k;
  void* pool_v;
  float* scale_k;
  float* scale_v;
  const int32_t* unit_table;
  int32_t* stamp;
  bf16_t* k_cmp;       // optional [1, NCB, H, D] pooled keys; page p of chunk cid -> row cid*ppc+p
  int64_t cs1, cs2;
  bf16_t* v_cmp;       // optional pooled values, same layout
  int64_t vcs1, vcs2;
  bf16_t* ring_k;      // optional bf16 copy of the chunk's keys [1, S, H, D] (a window ring slot)
  int64_t rks1, rks2;
  bf16_t* ring_v;      // optional copy of the values, same layout
  int64_t rvs1, rvs2;
  int H, D, P, ppc, max_chunks, cid, tokens, lph, epoch, n_slots;
};

__device__ __forceinline__ void unpack_bf16x8(const uint4& r, float (&f)[8]) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint2 quant8(const float (&x)[8], float inv) {
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = fminf(fmaxf(x[i] * inv, -448.0f), 448.0f);
  return make_uint2(f32x4_to_e4m3(y[0], y[1], y[2], y[3]), f32x4_to_e4m3(y[4], y[5], y[6], y[7]));
}

// 8 pooled sums / count, rounded to bf16 and packed (zeros for an empty page)
__device__ __forceinline__ uint4 mean8(const float (&sum)[8], float cnt, int n) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = n > 0 ? f32_to_bf16_bits(sum[2 * i] / cnt) : 0;
    const uint16_t hi = n > 0 ? f32_to_bf16_bits(sum[2 * i + 1] / cnt) : 0;
    w[i] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// One wave per (page, heads of the wave); lane = (head in wave, 8-dim slice).  Every lane walks
// the page's tokens in ascending order, so the pooled key is the omm_block_pool arithmetic; the
// walk loads kAppendBatch tokens of K and V at a time (all in flight together) and then adds them
// in order, so a lane waits for memory once per batch, not once per token.
constexpr int kAppendBatch = 16;

template <bool FP8>
__global__ __launch_bounds__(64) void paged_append_kernel(AppendArgs a) {
  const int lane = lane_id();
  const int hl = lane / a.lph, dc = lane - hl * a.lph;
  const int h = blockIdx.y * (kWave / a.lph) + hl;
  const int p = blockIdx.x;
  const bool active = hl < kWave / a.lph && h < a.H && dc * 8 < a.D;
  int32_t slot = -1;
  if (active) slot = a.unit_table[static_cast<int64_t>(h) * a.max_chunks + a.cid];
  const int t_first = p * a.P;
  const int nvalid = max(0, min(a.P, a.tokens - t_first));
  const bool go = active && slot >= 0 && slot < a.n_slots;
  const int64_t page = static_cast<int64_t>(slot) * a.ppc + p;
  const bf16_t* ksrc = a.k + static_cast<int64_t>(h) * a.ks2 + dc * 8;
  const bf16_t* vsrc = a.v + static_cast<int64_t>(h) * a.vs2 + dc * 8;
  constexpr int NB = kAppendBatch;
  // tokens t0 .. t0 + NB - 1 of the page (zeros past the valid ones)
  auto load_batch = [&](int t0, uint4 (&kr)[NB], uint4 (&vr)[NB]) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int t = t0 + j;
      kr[j] = vr[j] = make_uint4(0, 0, 0, 0);
      if (t < nvalid) {
        kr[j] = *reinterpret_cast<const uint4*>(ksrc + static_cast<int64_t>(t_first + t) * a.ks1);
        vr[j] = *reinterpret_cast<const uint4*>(vsrc + static_cast<int64_t>(t_first + t) * a.vs1);
      }
    }
  };

  float ksum[8], vsum[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ksum[i] = vsum[i] = 0.0f;

  if constexpr (!FP8) {
    uint4* kd = reinterpret_cast<uint4*>(static_cast<bf16_t*>(a.pool_k) + page * a.P * a.D + dc * 8);
    uint4* vd = reinterpret_cast<uint4*>(static_cast<bf16_t*>(a.pool_v) + page * a.P * a.D + dc * 8);
    const int64_t row = a.D / 8;  // uint4 per page row
    if (go) {
      for (int t0 = 0; t0 < a.P; t0 += NB) {
        uint4 kr[NB], vr[NB];
        load_batch(t0, kr, vr);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int t = t0 + j;
          if (t < nvalid) {
            float f[8], g[8];
            unpack_bf16x8(kr[j], f);
            unpack_bf16x8(vr[j], g);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              ksum[i] += f[i];
              vsum[i] += g[i];
            }
          }
          if (t < a.P) {
            kd[t * row] = kr[j];
            vd[t * row] = vr[j];
          }
        }
      }
    }
  } else {
    float amax_k = 0.0f, amax_v = 0.0f;
    if (go) {
      for (int t0 = 0; t0 < nvalid; t0 += NB) {
        uint4 kr[NB], vr[NB];
        load_batch(t0, kr, vr);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          if (t0 + j < nvalid) {
            float fk[8], fv[8];
            unpack_bf16x8(kr[j], fk);
            unpack_bf16x8(vr[j], fv);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              ksum[i] += fk[i];
              vsum[i] += fv[i];
              amax_k = fmaxf(amax_k, fabsf(fk[i]));
              amax_v = fmaxf(amax_v, fabsf(fv[i]));
            }
          }
        }
      }
    }
    // max over the lanes of one head (exact, order-free); all lanes take part in the shuffles
    for (int m = 1; m < a.lph; m <<= 1) {
      amax_k = fmaxf(amax_k, __shfl_xor(amax_k, m, kWave));
      amax_v = fmaxf(amax_v, __shfl_xor(amax_v, m, kWave));
    }
    if (go) {
      const float sk = amax_k > 0.0f ? amax_k / 448.0f : 1.0f;
      const float ik = amax_k > 0.0f ? 448.0f / amax_k : 1.0f;
      const float sv = amax_v > 0.0f ? amax_v / 448.0f : 1.0f;
      const float iv = amax_v > 0.0f ? 448.0f / amax_v : 1.0f;
      uint2* kd = reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.pool_k) + page * a.P * a.D + dc * 8);
      uint2* vd = reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.pool_v) + page * a.P * a.D + dc * 8);
      const int64_t row = a.D / 8;  // uint2 per page row
      // second pass over the page (its rows were just read: L2 hits)
      for (int t0 = 0; t0 < a.P; t0 += NB) {
        uint4 kr[NB], vr[NB];
        load_batch(t0, kr, vr);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int t = t0 + j;
          uint2 kq = make_uint2(0, 0), vq = make_uint2(0, 0);
          if (t < nvalid) {
            float fk[8], fv[8];
            unpack_bf16x8(kr[j], fk);
            unpack_bf16x8(vr[j], fv);
            kq = quant8(fk, ik);
            vq = quant8(fv, iv);
          }
          if (t < a.P) {
            kd[t * row] = kq;
            vd[t * row] = vq;
          }
        }
      }
      if (dc == 0) {
        a.scale_k[page] = sk;
        a.scale_v[page] = sv;
      }
    }
  }
  const float cnt = static_cast<float>(nvalid);
  const int64_t crow = static_cast<int64_t>(a.cid) * a.ppc + p;
  if (go && a.k_cmp != nullptr)
    *reinterpret_cast<uint4*>(a.k_cmp + crow * a.cs1 + h * a.cs2 + dc * 8) = mean8(ksum, cnt, nvalid);
  if (go && a.v_cmp != nullptr)
    *reinterpret_cast<uint4*>(a.v_cmp + crow * a.vcs1 + h * a.vcs2 + dc * 8) = mean8(vsum, cnt, nvalid);
  if (go && p == 0 && dc == 0 && a.stamp != nullptr && a.epoch > 0)
    a.stamp[static_cast<int64_t>(h) * a.max_chunks + a.cid] = a.epoch;
}

// The same append with a workgroup of 16 waves per (page, heads of a wave), for pages of at most
// 64 tokens: all 1024 threads load the page's K and V rows (16-byte columns c = tid % 64, rows
// tid / 64 + 16 j, every load of a thread in flight at once), write the bf16 pages straight from
// registers and stage the rows in LDS; then waves 0-3 (K) and 4-7 (V) add the staged rows in
// token order per element, so the pooled rows keep the omm_block_pool arithmetic.  fp8 pages take
// the per-(page, head) amax from the registers (wave shuffles, then a 16-wave LDS reduction) and
// quantise the registers: one read of the chunk.  The whole chunk is in flight at once (222
// workgroups x 1024 threads x 8 loads); a wave moves a bounded number of bytes at a time, so the
// same loads spread over 16 waves per page instead of 4 finish sooner, and the pooled sums over 8
// waves instead of 2 (AR chunk, graph replay: 12.3 against 14.7 us bf16, 11.7 against 14.4 us
// fp8).
constexpr int kAppendThreads = 1024;
constexpr int kAppendWaves = kAppendThreads / kWave;
constexpr int kAppendMaxP = 64;
constexpr int kAppendRows = kAppendMaxP / kAppendWaves;  // rows per thread (4)

template <bool FP8>
__global__ __launch_bounds__(kAppendThreads) void paged_append_wg_kernel(AppendArgs a) {
  extern __shared__ __align__(16) uint4 stage[];  // [2][P][64]: K rows, then V rows
  __shared__ float amx[2][kAppendThreads / kWave][kWave];
  const int tid = threadIdx.x, w = tid / kWave, lane = lane_id();
  const int c = lane, hl = c / a.lph, dc = c - hl * a.lph;
  const int hpw = kWave / a.lph;  // heads per wave (lph divides 64)
  const int h = blockIdx.y * hpw + hl;
  const int p = blockIdx.x;
  const int P = a.P;
  const bool col_ok = h < a.H;
  int32_t slot = -1;
  if (col_ok) slot = a.unit_table[static_cast<int64_t>(h) * a.max_chunks + a.cid];
  const bool go = col_ok && slot >= 0 && slot < a.n_slots;
  const int t_first = p * P;
  const int nvalid = max(0, min(P, a.tokens - t_first));
  const int64_t page = static_cast<int64_t>(slot) * a.ppc + p;
  const bf16_t* ksrc = a.k + static_cast<int64_t>(h) * a.ks2 + dc * 8;
  const bf16_t* vsrc = a.v + static_cast<int64_t>(h) * a.vs2 + dc * 8;
  constexpr int NR = kAppendRows;
  uint4 kr[NR], vr[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int r = w + kAppendWaves * j;
    kr[j] = vr[j] = make_uint4(0, 0, 0, 0);
    if (go && r < nvalid) {
      kr[j] = *reinterpret_cast<const uint4*>(ksrc + static_cast<int64_t>(t_first + r) * a.ks1);
      vr[j] = *reinterpret_cast<const uint4*>(vsrc + static_cast<int64_t>(t_first + r) * a.vs1);
    }
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int r = w + kAppendWaves * j;
    if (r < nvalid) {
      stage[r * kWave + c] = kr[j];
      stage[(P + r) * kWave + c] = vr[j];
    }
  }
  if constexpr (!FP8) {
    if (go) {
      uint4* kd = reinterpret_cast<uint4*>(static_cast<bf16_t*>(a.pool_k) + page * P * a.D + dc * 8);
      uint4* vd = reinterpret_cast<uint4*>(static_cast<bf16_t*>(a.pool_v) + page * P * a.D + dc * 8);
      const int64_t row = a.D / 8;
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const int r = w + kAppendWaves * j;
        if (r < P) {
          kd[r * row] = kr[j];
          vd[r * row] = vr[j];
        }
      }
    }
  } else {
    float mk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      float fk[8], fv[8];
      unpack_bf16x8(kr[j], fk);
      unpack_bf16x8(vr[j], fv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        mk = fmaxf(mk, fabsf(fk[i]));
        mv = fmaxf(mv, fabsf(fv[i]));
      }
    }
    // max over the lanes of one head in this wave (exact, order-free), then over the 4 waves
    for (int m = 1; m < a.lph; m <<= 1) {
      mk = fmaxf(mk, __shfl_xor(mk, m, kWave));
      mv = fmaxf(mv, __shfl_xor(mv, m, kWave));
    }
    amx[0][w][lane] = mk;
    amx[1][w][lane] = mv;
    __syncthreads();
#pragma unroll
    for (int ww = 0; ww < kAppendThreads / kWave; ++ww) {
      mk = fmaxf(mk, amx[0][ww][lane]);
      mv = fmaxf(mv, amx[1][ww][lane]);
    }
    if (go) {
      const float ik = mk > 0.0f ? 448.0f / mk : 1.0f;
      const float iv = mv > 0.0f ? 448.0f / mv : 1.0f;
      uint2* kd = reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.pool_k) + page * P * a.D + dc * 8);
      uint2* vd = reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.pool_v) + page * P * a.D + dc * 8);
      const int64_t row = a.D / 8;
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const int r = w + kAppendWaves * j;
        if (r < P) {
          uint2 kq = make_uint2(0, 0), vq = make_uint2(0, 0);
          if (r < nvalid) {
            float fk[8], fv[8];
            unpack_bf16x8(kr[j], fk);
            unpack_bf16x8(vr[j], fv);
            kq = quant8(fk, ik);
            vq = quant8(fv, iv);
          }
          kd[r * row] = kq;
          vd[r * row] = vq;
        }
      }
      if (w == 0 && dc == 0) {
        a.scale_k[page] = mk > 0.0f ? mk / 448.0f : 1.0f;
        a.scale_v[page] = mv > 0.0f ? mv / 448.0f : 1.0f;
      }
    }
  }
  __syncthreads();
  // pooled rows: waves 0-3 add the K rows, waves 4-7 the V rows; wave w takes elements 2 (w % 4)
  // and 2 (w % 4) + 1 of every 16-byte column, each in token order (the omm_block_pool sum)
  if (w < 8 && go) {
    const bool isv = w >= 4;
    const int e2 = w & 3;  // element pair of the column
    const uint32_t* src = reinterpret_cast<const uint32_t*>(stage + (isv ? P * kWave : 0) + c) + e2;
    float s0 = 0.0f, s1 = 0.0f;
    int r = 0;
    for (; r + 16 <= nvalid; r += 16) {
      uint32_t x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = src[(r + u) * kWave * 4];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        s0 += bf16_bits_to_f32(static_cast<uint16_t>(x[u]));
        s1 += bf16_bits_to_f32(static_cast<uint16_t>(x[u] >> 16));
      }
    }
    for (; r < nvalid; ++r) {
      const uint32_t x = src[r * kWave * 4];
      s0 += bf16_bits_to_f32(static_cast<uint16_t>(x));
      s1 += bf16_bits_to_f32(static_cast<uint16_t>(x >> 16));
    }
    const float cnt = static_cast<float>(nvalid);
    const uint16_t lo = nvalid > 0 ? f32_to_bf16_bits(s0 / cnt) : 0;
    const uint16_t hi = nvalid > 0 ? f32_to_bf16_bits(s1 / cnt) : 0;
    const uint32_t packed = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    const int64_t crow = static_cast<int64_t>(a.cid) * a.ppc + p;
    bf16_t* dst = isv ? a.v_cmp : a.k_cmp;
    if (dst != nullptr) {
      const int64_t off = isv ? crow * a.vcs1 + h * a.vcs2 : crow * a.cs1 + h * a.cs2;
      *reinterpret_cast<uint32_t*>(dst + off + dc * 8 + 2 * e2) = packed;
    }
  }
  if (go && w == 0 && p == 0 && dc == 0 && a.stamp != nullptr && a.epoch > 0)
    a.stamp[static_cast<int64_t>(h) * a.max_chunks + a.cid] = a.epoch;
}

// The same append with one workgroup of 4 waves per (page, head, K or V), for pages of at most
// 64 tokens and head dims of 64 or 128 (kAppHeadThreads threads; blockIdx.z = 0 for K, 1 for V;
// the AR chunk: 74 x 12 x 2 = 1,776 workgroups, several per CU).  Lane (tl, dc): a wave's load
// covers TPI = 64 / lph consecutive token rows of the head, 16 bytes per lane; the thread's rows
// are TPI (w + 4 j) + tl.  bf16 pages are written from registers.  fp8 takes the page's amax
// over the whole wave (one head) and the 4 waves through LDS, so the one barrier that holds the
// stores spans 4 waves and one tensor; that barrier also publishes the LDS-staged rows, from
// which one thread per element pair adds the pooled row in token order.  AR chunk, graph replay:
// bf16 11.0 us, fp8 9.7-9.9 us, against 11.3 / 10.5-10.7 with K and V of a (page, head) in one
// workgroup and 11.7 / 12.1 with 16-wave (page, 4 heads) workgroups.  Measured and not kept: 2 or
// 8 waves per workgroup (fp8 10.4 / 10.5 us), one thread per pooled element, and persistent
// workgroups that load the next item while storing the current one (11.5-16.3 us fp8): the
// chunk's loads all in flight at once is fastest.
constexpr int kAppHeadThreads = 256;
constexpr int kAppHeadWaves = kAppHeadThreads / kWave;

template <bool FP8>
__global__ __launch_bounds__(kAppHeadThreads) void paged_append_kv_kernel(AppendArgs a) {
  __shared__ __align__(16) uint4 stage[kAppendMaxP][16];  // [token row][16-byte column]
  __shared__ float amx[kAppHeadWaves];
  const int tid = threadIdx.x, w = tid / kWave, lane = lane_id();
  const int lph = a.lph, TPI = kWave / lph;
  const int tl = lane / lph, dc = lane - tl * lph;
  const int p = blockIdx.x, h = blockIdx.y;
  const bool isv = blockIdx.z != 0;
  const int32_t slot = a.unit_table[static_cast<int64_t>(h) * a.max_chunks + a.cid];
  const bool pages = slot >= 0 && slot < a.n_slots;  // no unit slot: only the ring is written
  bf16_t* ring = isv ? a.ring_v : a.ring_k;
  if (!pages && ring == nullptr) return;  // whole workgroup
  const int P = a.P;
  const int t_first = p * P;
  const int nvalid = max(0, min(P, a.tokens - t_first));
  const int64_t page = static_cast<int64_t>(slot) * a.ppc + p;
  const bf16_t* src = (isv ? a.v + static_cast<int64_t>(h) * a.vs2 : a.k + static_cast<int64_t>(h) * a.ks2) + dc * 8;
  const int64_t s1 = isv ? a.vs1 : a.ks1;
  constexpr int NR = kAppendMaxP / (kAppHeadWaves * 4);
  uint4 xr[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int r = TPI * (w + kAppHeadWaves * j) + tl;
    xr[j] = make_uint4(0, 0, 0, 0);
    if (r < nvalid) xr[j] = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(t_first + r) * s1);
  }
  if (ring != nullptr) {  // the chunk's bf16 rows, copied from registers
    const int64_t rs1 = isv ? a.rvs1 : a.rks1;
    ring += static_cast<int64_t>(h) * (isv ? a.rvs2 : a.rks2) + dc * 8;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int r = TPI * (w + kAppHeadWaves * j) + tl;
      if (r < nvalid) *reinterpret_cast<uint4*>(ring + static_cast<int64_t>(t_first + r) * rs1) = xr[j];
    }
  }
  if (!pages) return;  // whole workgroup
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int r = TPI * (w + kAppHeadWaves * j) + tl;
    if (r < nvalid) stage[r][dc] = xr[j];
  }
  const int64_t row = a.D / 8;
  if constexpr (!FP8) {
    uint4* d = reinterpret_cast<uint4*>(static_cast<bf16_t*>(isv ? a.pool_v : a.pool_k) + page * P * a.D + dc * 8);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int r = TPI * (w + kAppHeadWaves * j) + tl;
      if (r < P) d[r * row] = xr[j];
    }
    __syncthreads();
  } else {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      float f[8];
      unpack_bf16x8(xr[j], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(f[i]));
    }
#pragma unroll
    for (int mm = 1; mm < kWave; mm <<= 1) m = fmaxf(m, __shfl_xor(m, mm, kWave));
    if (lane == 0) amx[w] = m;
    __syncthreads();
#pragma unroll
    for (int ww = 0; ww < kAppHeadWaves; ++ww) m = fmaxf(m, amx[ww]);
    const float im = m > 0.0f ? 448.0f / m : 1.0f;
    uint2* d = reinterpret_cast<uint2*>(static_cast<uint8_t*>(isv ? a.pool_v : a.pool_k) + page * P * a.D + dc * 8);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int r = TPI * (w + kAppHeadWaves * j) + tl;
      if (r < P) {
        uint2 qv = make_uint2(0, 0);
        if (r < nvalid) {
          float f[8];
          unpack_bf16x8(xr[j], f);
          qv = quant8(f, im);
        }
        d[r * row] = qv;
      }
    }
    if (tid == 0) (isv ? a.scale_v : a.scale_k)[page] = m > 0.0f ? m / 448.0f : 1.0f;
  }
  // pooled row: thread t < D / 2 takes element pair t, adding the staged rows in token order
  if (tid < a.D / 2) {
    const int e = tid;
    const int col = e >> 2, e2 = e & 3;
    const uint32_t* sp = reinterpret_cast<const uint32_t*>(&stage[0][col]) + e2;
    constexpr int RS = 16 * 4;
    float s0 = 0.0f, s1f = 0.0f;
    int r = 0;
    for (; r + 16 <= nvalid; r += 16) {
      uint32_t x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = sp[(r + u) * RS];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        s0 += bf16_bits_to_f32(static_cast<uint16_t>(x[u]));
        s1f += bf16_bits_to_f32(static_cast<uint16_t>(x[u] >> 16));
      }
    }
    for (; r < nvalid; ++r) {
      const uint32_t x = sp[r * RS];
      s0 += bf16_bits_to_f32(static_cast<uint16_t>(x));
      s1f += bf16_bits_to_f32(static_cast<uint16_t>(x >> 16));
    }
    const float cnt = static_cast<float>(nvalid);
    const uint16_t lo = nvalid > 0 ? f32_to_bf16_bits(s0 / cnt) : 0;
    const uint16_t hi = nvalid > 0 ? f32_to_bf16_bits(s1f / cnt) : 0;
    const uint32_t packed = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    const int64_t crow = static_cast<int64_t>(a.cid) * a.ppc + p;
    bf16_t* dst = isv ? a.v_cmp : a.k_cmp;
    if (dst != nullptr) {
      const int64_t off = isv ? crow * a.vcs1 + h * a.vcs2 : crow * a.cs1 + h * a.cs2;
      *reinterpret_cast<uint32_t*>(dst + off + 2 * e) = packed;
    }
  }
  if (!isv && p == 0 && tid == 0 && a.stamp != nullptr && a.epoch > 0)
    a.stamp[static_cast<int64_t>(h) * a.max_chunks + a.cid] = a.epoch;
}


// ---- batched unit copies (evict to the host pool, promote to HBM) ---------------------------
constexpr int64_t kCopyPart = 64 * 1024;  // bytes per workgroup

struct CopyArgs {
  const unsigned char* src_k;
  unsigned char* dst_k;
  const unsigned char* src_v;
  unsigned char* dst_v;
  const unsigned char* src_sk;
  unsigned char* dst_sk;
  const unsigned char* src_sv;
  unsigned char* dst_sv;
  const int32_t* src_slot;
  const int32_t* dst_slot;
  int64_t unit_bytes, scale_bytes;
  int32_t n_src, n_dst;  // slots in the source / destination pools
};

__device__ __forceinline__ void copy_range16(const unsigned char* s, unsigned char* d, int64_t n) {
  const uint4* s4 = reinterpret_cast<const uint4*>(s);
  uint4* d4 = reinterpret_cast<uint4*>(d);
  const int64_t n4 = n / 16;
  const int64_t st = blockDim.x;
  int64_t i = threadIdx.x;
  // four 16-byte loads in flight per lane
  for (; i + 3 * st < n4; i += 4 * st) {
    const uint4 r0 = s4[i], r1 = s4[i + st], r2 = s4[i + 2 * st], r3 = s4[i + 3 * st];
    d4[i] = r0;
    d4[i + st] = r1;
    d4[i + 2 * st] = r2;
    d4[i + 3 * st] = r3;
  }
  for (; i < n4; i += st) d4[i] = s4[i];
}

__global__ __launch_bounds__(256) void copy_units_kernel(CopyArgs a) {
  const int64_t i = blockIdx.x;
  const int64_t part = blockIdx.y;
  const int64_t so = static_cast<int64_t>(a.src_slot[i]), dof = static_cast<int64_t>(a.dst_slot[i]);
  if (so < 0 || so >= a.n_src || dof < 0 || dof >= a.n_dst) return;  // workgroup-uniform
  const int64_t b0 = part * kCopyPart;
  const int64_t n = min(kCopyPart, a.unit_bytes - b0);
  if (n > 0) {
    copy_range16(a.src_k + so * a.unit_bytes + b0, a.dst_k + dof * a.unit_bytes + b0, n);
    if (a.src_v != nullptr)
      copy_range16(a.src_v + so * a.unit_bytes + b0, a.dst_v + dof * a.unit_bytes + b0, n);
  }
  if (part == 0 && a.scale_bytes > 0) {
    for (int64_t j = threadIdx.x; j < a.scale_bytes; j += blockDim.x) {
      if (a.src_sk != nullptr) a.dst_sk[dof * a.scale_bytes + j] = a.src_sk[so * a.scale_bytes + j];
      if (a.src_sv != nullptr) a.dst_sv[dof * a.scale_bytes + j] = a.src_sv[so * a.scale_bytes + j];
    }
  }
}

// ---- K1: gather + publish + clear -----------------------------------------------------------
constexpr int kClearPerWg = 256;

__device__ __forceinline__ void copy_bytes_wg(int64_t src, int64_t dst, int64_t nbytes) {
  if ((nbytes & 15) == 0 && ((src | dst) & 15) == 0) {
    copy_range16(reinterpret_cast<const unsigned char*>(src), reinterpret_cast<unsigned char*>(dst),
                 nbytes);
  } else {
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src);
    uint16_t* d = reinterpret_cast<uint16_t*>(dst);
    for (int64_t j = threadIdx.x; j < nbytes / 2; j += blockDim.x) d[j] = s[j];
  }
}

// desc has no __restrict__: the kernel stores through addresses read out of it
__global__ __launch_bounds__(256) void gather_publish_clear_kernel(const int64_t* desc,
                                                                   int64_t n_fetch,
                                                                   int64_t n_clear,
                                                                   int64_t block_bytes) {
  const int64_t w = blockIdx.x;
  if (w < n_fetch) {
    const int64_t sk = desc[w], sv = desc[n_fetch + w];
    const int64_t dk = desc[2 * n_fetch + w], dv = desc[3 * n_fetch + w];
    const int64_t pk = desc[4 * n_fetch + w], pv = desc[5 * n_fetch + w];
    copy_bytes_wg(sk, dk, block_bytes);
    copy_bytes_wg(sv, dv, block_bytes);
    __syncthreads();  // every lane's share of K and V is written before the addresses publish
    if (threadIdx.x == 0) {
      __threadfence();
      *reinterpret_cast<int64_t*>(pk) = dk;
      *reinterpret_cast<int64_t*>(pv) = dv;
    }
  } else {
    const int64_t base = (w - n_fetch) * kClearPerWg;
    for (int64_t j = threadIdx.x; j < kClearPerWg; j += blockDim.x) {
      const int64_t e = base + j;
      if (e < n_clear) *reinterpret_cast<int64_t*>(desc[6 * n_fetch + e]) = 0;
    }
  }
}

// ---- K2: table range register / clear ------------------------------------------------------
__global__ __launch_bounds__(128) void block_range_kernel(int64_t* table, int32_t* n_valid,
                                                          int64_t heads, int64_t mb,
                                                          int64_t first, int64_t n,
                                                          int64_t k_base, int64_t v_base,
                                                          int64_t head_stride, int64_t block_bytes,
                                                          int64_t n_valid_value, int write_k,
                                                          int write_v, int clear) {
  const int64_t h = blockIdx.x;
  const int64_t j = static_cast<int64_t>(blockIdx.y) * blockDim.x + threadIdx.x;
  if (j < n) {
    const int64_t off = h * head_stride + j * block_bytes;
    if (write_k) table[h * mb + first + j] = clear ? 0 : k_base + off;
    if (write_v) table[(heads + h) * mb + first + j] = clear ? 0 : v_base + off;
  }
  if (blockIdx.y == 0 && threadIdx.x == 0 && n_valid_value >= 0)
    n_valid[h] = static_cast<int32_t>(n_valid_value);
}

// ---- K3: dedup of selected (head, block) keys -----------------------------------------------
constexpr int kDedupTile = 1024;
constexpr int kDedupThreads = 256;
constexpr int kDedupMaxTiles = 1 << 15;

__global__ __launch_bounds__(256) void dedup_mark_kernel(const int32_t* __restrict__ ids,
                                                         int64_t n, int32_t* __restrict__ stamp,
                                                         int32_t epoch, int32_t mb, int32_t heads,
                                                         int32_t t, int32_t bpc) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t bid = ids[e];
    if (bid < 0 || bid >= mb) continue;
    const int32_t h = static_cast<int32_t>((e / t) % heads);
    const int32_t cid = bid / bpc, loc = bid - cid * bpc;
    stamp[(static_cast<int64_t>(cid) * heads + h) * bpc + loc] = epoch;  // duplicates agree
  }
}

// hits of one 1024-key tile; thread j owns keys 4j..4j+3
__device__ __forceinline__ int tile_hits(const int32_t* stamp, int64_t key0, int64_t n_keys,
                                         int32_t epoch, bool (&hit)[4]) {
  int c = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t key = key0 + 4 * threadIdx.x + i;
    hit[i] = key < n_keys && stamp[key] == epoch;
    c += hit[i] ? 1 : 0;
  }
  return c;
}

// exclusive prefix of v over the workgroup (256 threads, wave64); returns the total via *total
__device__ __forceinline__ int wg_exclusive_scan(int v, int* lds, int* total) {
  const int lane = lane_id(), w = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const int y = __shfl_up(x, m, kWave);
    if (lane >= m) x += y;
  }
  if (lane == kWave - 1) lds[w] = x;
  __syncthreads();
  int off = 0, tot = 0;
  for (int i = 0; i < kDedupThreads / kWave; ++i) {
    const int s = lds[i];
    if (i < w) off += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return off + x - v;
}

__global__ __launch_bounds__(256) void dedup_count_kernel(const int32_t* __restrict__ stamp,
                                                          int32_t* __restrict__ counts,
                                                          int64_t n_keys, int32_t epoch) {
  __shared__ int lds[kDedupThreads / kWave];
  bool hit[4];
  const int c = tile_hits(stamp, static_cast<int64_t>(blockIdx.x) * kDedupTile, n_keys, epoch, hit);
  int total;
  wg_exclusive_scan(c, lds, &total);
  if (threadIdx.x == 0) counts[blockIdx.x] = total;
}

__global__ __launch_bounds__(256) void dedup_scan_kernel(const int32_t* __restrict__ counts,
                                                         int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ out, int n_tiles) {
  __shared__ int lds[kDedupThreads / kWave];
  const int per = (n_tiles + kDedupThreads - 1) / kDedupThreads;
  const int b = threadIdx.x * per, e = min(b + per, n_tiles);
  int s = 0;
  for (int j = b; j < e; ++j) s += counts[j];
  int total;
  int run = wg_exclusive_scan(s, lds, &total);
  for (int j = b; j < e; ++j) {
    offsets[j] = run;
    run += counts[j];
  }
  if (threadIdx.x == 0) out[0] = total;
}

__global__ __launch_bounds__(256) void dedup_compact_kernel(const int32_t* __restrict__ stamp,
                                                            const int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ out,
                                                            int64_t n_keys, int64_t cap,
                                                            int32_t epoch) {
  __shared__ int lds[kDedupThreads / kWave];
  bool hit[4];
  const int64_t key0 = static_cast<int64_t>(blockIdx.x) * kDedupTile;
  const int c = tile_hits(stamp, key0, n_keys, epoch, hit);
  int total;
  int pos = offsets[blockIdx.x] + wg_exclusive_scan(c, lds, &total);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (hit[i]) {
      if (pos < cap) out[1 + pos] = static_cast<int32_t>(key0 + 4 * threadIdx.x + i);
      ++pos;
    }
  }
}

int check_view_i32(const omm_view4* v, const char* what) {
  OMM_REQUIRE(v != nullptr, OMM_EINVAL, "%s: null view", what);
  for (int i = 0; i < 4; ++i)
    OMM_REQUIRE(v->size[i] >= 0 && v->stride[i] >= 0, OMM_EINVAL, "%s: negative size or stride", what);
  return OMM_OK;
}

}  // namespace
}  // namespace omm

extern "C" int omm_build_ptr_table(const omm_view4* ids, const int64_t* base_k,
                                   const int64_t* base_v, int64_t base_stride_h,
                                   int64_t base_stride_c, int32_t max_chunks,
                                   const int32_t* n_blocks_per_head, int64_t batch_stride,
                                   int32_t blocks_per_chunk, int64_t in_chunk_block_bytes,
                                   int64_t* ptr_k, int64_t* ptr_v, void* stream) {
  using namespace omm;
  int rc = check_view_i32(ids, "omm_build_ptr_table");
  if (rc) return rc;
  OMM_REQUIRE(blocks_per_chunk >= 0, OMM_EINVAL, "omm_build_ptr_table: blocks_per_chunk must be >= 0");
  OMM_REQUIRE(blocks_per_chunk == 0 || in_chunk_block_bytes > 0, OMM_EINVAL,
              "omm_build_ptr_table: in_chunk_block_bytes required for a chunk-level base table");
  const int64_t total = ids->size[0] * ids->size[1] * ids->size[2] * ids->size[3];
  if (total == 0) return OMM_OK;
  OMM_REQUIRE(max_chunks > 0, OMM_EINVAL, "omm_build_ptr_table: empty base table");
  OMM_REQUIRE(ids->data && base_k && base_v && n_blocks_per_head && ptr_k && ptr_v, OMM_EINVAL,
              "omm_build_ptr_table: null pointer");
  OMM_REQUIRE(ids->size[1] <= 2147483647ll && ids->size[2] <= 2147483647ll &&
                  ids->size[3] <= 2147483647ll,
              OMM_EUNSUPPORTED, "omm_build_ptr_table: dimension too large");
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv64(total, 256), 65535));
  ptr_table_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const int32_t*>(ids->data), ids->stride[0], ids->stride[1], ids->stride[2],
      ids->stride[3], base_k, base_v, base_stride_h, base_stride_c, max_chunks, n_blocks_per_head,
      ptr_k, ptr_v, static_cast<int>(ids->size[1]), static_cast<int>(ids->size[2]),
      static_cast<int>(ids->size[3]), batch_stride, blocks_per_chunk, in_chunk_block_bytes, total);
  return check_launch("omm_build_ptr_table");
}

namespace omm {
namespace {
int check_cmp(const omm_view4* c, int64_t rows, int H, int D, const char* what) {
  OMM_REQUIRE(c->size[0] == 1 && c->size[1] >= rows && c->size[2] == H && c->size[3] == D &&
                  c->stride[3] == 1 && c->stride[1] % 8 == 0 && c->stride[2] % 8 == 0 &&
                  (reinterpret_cast<uintptr_t>(c->data) & 15u) == 0,
              OMM_EINVAL, "omm_paged_append: %s must be a 16-byte aligned [1, >= %lld, %d, %d] bf16 view",
              what, (long long)rows, H, D);
  return OMM_OK;
}

// The bf16 ring copy for the append kernels that do not write it themselves: one 16-byte piece
// of one (token, head) row per thread.
__global__ __launch_bounds__(256) void ring_copy_kernel(const bf16_t* __restrict__ src,
                                                        int64_t ss1, int64_t ss2,
                                                        bf16_t* __restrict__ dst, int64_t ds1,
                                                        int64_t ds2, int S, int H, int D8) {
  const int64_t n = static_cast<int64_t>(S) * H * D8;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int c = static_cast<int>(i % D8);
    const int64_t r = i / D8;
    const int h = static_cast<int>(r % H);
    const int64_t t = r / H;
    *reinterpret_cast<uint4*>(dst + t * ds1 + h * ds2 + 8 * c) =
        *reinterpret_cast<const uint4*>(src + t * ss1 + h * ss2 + 8 * c);
  }
}
}  // namespace
}  // namespace omm

extern "C" int omm_paged_append(const omm_paged_kv* kv, const omm_view4* k_new,
                                const omm_view4* v_new, int32_t cid, int32_t chunk_tokens,
                                const omm_view4* k_cmp, const omm_view4* v_cmp, int32_t epoch,
                                void* stream) {
  return omm_paged_append_ring(kv, k_new, v_new, cid, chunk_tokens, k_cmp, v_cmp, nullptr,
                               nullptr, epoch, stream);
}

extern "C" int omm_paged_append_ring(const omm_paged_kv* kv, const omm_view4* k_new,
                                     const omm_view4* v_new, int32_t cid, int32_t chunk_tokens,
                                     const omm_view4* k_cmp, const omm_view4* v_cmp,
                                     const omm_view4* ring_k, const omm_view4* ring_v,
                                     int32_t epoch, void* stream) {
  using namespace omm;
  OMM_REQUIRE(kv != nullptr && k_new != nullptr && v_new != nullptr, OMM_EINVAL,
              "omm_paged_append: null argument");
  const int H = kv->num_heads, D = kv->head_dim, P = kv->page_tokens, ppc = kv->pages_per_chunk;
  OMM_REQUIRE(kv->dtype == OMM_BF16 || kv->dtype == OMM_FP8E4M3, OMM_EINVAL,
              "omm_paged_append: cache dtype must be bf16 or fp8e4m3");
  OMM_REQUIRE(H >= 1 && D >= 8 && D <= 256 && D % 8 == 0 && P >= 1 && kv->chunk_len >= 1 &&
                  ppc == cdiv64(kv->chunk_len, P),
              OMM_EINVAL, "omm_paged_append: inconsistent cache geometry");
  OMM_REQUIRE(cid >= 0 && cid < kv->max_chunks, OMM_EINVAL,
              "omm_paged_append: chunk id %d outside [0, %d)", cid, kv->max_chunks);
  // Whole chunks only: attention reads every page of a written chunk with the token counts
  // chunk_len fixes (the last page's tail past chunk_len is the only padding), so a shorter
  // write would expose unwritten slots to the softmax.
  OMM_REQUIRE(chunk_tokens == kv->chunk_len, OMM_EINVAL,
              "omm_paged_append: %d tokens for a chunk of %d (whole chunks only)", chunk_tokens,
              kv->chunk_len);
  for (const omm_view4* x : {k_new, v_new}) {
    OMM_REQUIRE(x->size[0] == 1 && x->size[1] == chunk_tokens && x->size[2] == H &&
                    x->size[3] == D,
                OMM_EINVAL, "omm_paged_append: k_new / v_new must be [1, %d, %d, %d]", chunk_tokens,
                H, D);
    OMM_REQUIRE(x->stride[3] == 1 && x->stride[1] % 8 == 0 && x->stride[2] % 8 == 0 &&
                    (reinterpret_cast<uintptr_t>(x->data) & 15u) == 0,
                OMM_EUNSUPPORTED,
                "omm_paged_append: k_new / v_new need unit dim stride and 16-byte aligned rows");
  }
  OMM_REQUIRE(kv->pool_k && kv->pool_v && kv->unit_table, OMM_EINVAL, "omm_paged_append: null pool");
  OMM_REQUIRE(kv->dtype == OMM_BF16 || (kv->scale_k && kv->scale_v), OMM_EINVAL,
              "omm_paged_append: fp8 cache without scale arrays");
  AppendArgs a{};
  a.k = static_cast<const bf16_t*>(k_new->data);
  a.v = static_cast<const bf16_t*>(v_new->data);
  a.ks1 = k_new->stride[1]; a.ks2 = k_new->stride[2];
  a.vs1 = v_new->stride[1]; a.vs2 = v_new->stride[2];
  a.pool_k = kv->pool_k; a.pool_v = kv->pool_v;
  a.scale_k = kv->scale_k; a.scale_v = kv->scale_v;
  a.unit_table = kv->unit_table;
  a.stamp = kv->stamp;
  const int64_t rows = static_cast<int64_t>(cid + 1) * ppc;
  if (k_cmp != nullptr && k_cmp->data != nullptr) {
    const int rc = check_cmp(k_cmp, rows, H, D, "k_cmp");
    if (rc) return rc;
    a.k_cmp = static_cast<bf16_t*>(const_cast<void*>(k_cmp->data));
    a.cs1 = k_cmp->stride[1]; a.cs2 = k_cmp->stride[2];
  }
  if (v_cmp != nullptr && v_cmp->data != nullptr) {
    const int rc = check_cmp(v_cmp, rows, H, D, "v_cmp");
    if (rc) return rc;
    a.v_cmp = static_cast<bf16_t*>(const_cast<void*>(v_cmp->data));
    a.vcs1 = v_cmp->stride[1]; a.vcs2 = v_cmp->stride[2];
  }
  // ring copies: [1, chunk_tokens, H, D] bf16 views with unit dim stride and 16-byte rows, apart
  // from the inputs (the copy is written while they are read)
  for (const omm_view4* r : {ring_k, ring_v}) {
    if (r == nullptr || r->data == nullptr) continue;
    OMM_REQUIRE(r->size[0] == 1 && r->size[1] == chunk_tokens && r->size[2] == H &&
                    r->size[3] == D && r->stride[3] == 1 && r->stride[1] % 8 == 0 &&
                    r->stride[2] % 8 == 0 && (reinterpret_cast<uintptr_t>(r->data) & 15u) == 0,
                OMM_EINVAL,
                "omm_paged_append: ring_k / ring_v must be 16-byte aligned [1, %d, %d, %d] bf16 "
                "views with unit dim stride", chunk_tokens, H, D);
    OMM_REQUIRE(!views_overlap(*r, *k_new, 2) && !views_overlap(*r, *v_new, 2), OMM_EINVAL,
                "omm_paged_append: a ring view overlaps k_new / v_new");
  }
  if (ring_k != nullptr && ring_k->data != nullptr) {
    a.ring_k = static_cast<bf16_t*>(const_cast<void*>(ring_k->data));
    a.rks1 = ring_k->stride[1]; a.rks2 = ring_k->stride[2];
  }
  if (ring_v != nullptr && ring_v->data != nullptr) {
    a.ring_v = static_cast<bf16_t*>(const_cast<void*>(ring_v->data));
    a.rvs1 = ring_v->stride[1]; a.rvs2 = ring_v->stride[2];
  }
  a.H = H; a.D = D; a.P = P; a.ppc = ppc; a.max_chunks = kv->max_chunks; a.cid = cid;
  a.tokens = chunk_tokens;
  a.n_slots = kv->n_slots;
  a.lph = D / 8;
  a.epoch = epoch;
  // lanes per head must divide the wave
  OMM_REQUIRE(kWave % a.lph == 0, OMM_EUNSUPPORTED, "omm_paged_append: head dim %d", D);
  const dim3 grid(static_cast<unsigned>(ppc), static_cast<unsigned>(cdiv64(H, kWave / a.lph)));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (P <= kAppendMaxP && (D == 64 || D == 128)) {
    const dim3 hgrid(static_cast<unsigned>(ppc), static_cast<unsigned>(H), 2u);
    if (kv->dtype == OMM_BF16)
      paged_append_kv_kernel<false><<<hgrid, kAppHeadThreads, 0, s>>>(a);
    else
      paged_append_kv_kernel<true><<<hgrid, kAppHeadThreads, 0, s>>>(a);
    return check_launch("omm_paged_append");
  }
  // the other append kernels leave the ring copies to ring_copy_kernel
  for (int t = 0; t < 2; ++t) {
    bf16_t* ring = t == 0 ? a.ring_k : a.ring_v;
    if (ring == nullptr) continue;
    const int64_t n = static_cast<int64_t>(chunk_tokens) * H * (D / 8);
    const unsigned blocks = static_cast<unsigned>(n / 256 + 1 < 4096 ? n / 256 + 1 : 4096);
    ring_copy_kernel<<<blocks, 256, 0, s>>>(t == 0 ? a.k : a.v, t == 0 ? a.ks1 : a.vs1,
                                            t == 0 ? a.ks2 : a.vs2, ring,
                                            t == 0 ? a.rks1 : a.rvs1, t == 0 ? a.rks2 : a.rvs2,
                                            chunk_tokens, H, D / 8);
  }
  if (P <= kAppendMaxP) {
    const size_t lds = static_cast<size_t>(2) * P * kWave * sizeof(uint4);
    const void* fn = kv->dtype == OMM_BF16
                         ? reinterpret_cast<const void*>(&paged_append_wg_kernel<false>)
                         : reinterpret_cast<const void*>(&paged_append_wg_kernel<true>);
    if (lds > 64 * 1024) {
      const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               static_cast<int>(lds));
      OMM_REQUIRE(e == hipSuccess, OMM_EHIP, "omm_paged_append: LDS attribute: %s",
                  hipGetErrorString(e));
    }
    if (kv->dtype == OMM_BF16)
      paged_append_wg_kernel<false><<<grid, kAppendThreads, lds, s>>>(a);
    else
      paged_append_wg_kernel<true><<<grid, kAppendThreads, lds, s>>>(a);
    return check_launch("omm_paged_append");
  }
  if (kv->dtype == OMM_BF16)
    paged_append_kernel<false><<<grid, kWave, 0, s>>>(a);
  else
    paged_append_kernel<true><<<grid, kWave, 0, s>>>(a);
  return check_launch("omm_paged_append");
}

namespace omm {
namespace {
// ---- staging of host-resident pages for one selection call ------------------------------------
// A grid of kStageWaves one-wave workgroups strides over the (query group, head) rows of ids,
// one row per wave at a time.  The kernel runs beside the attention kernels of the same layer;
// 128 waves keep the host link busy while holding few wave slots (one wave per row, 888 rows in
// the AR shape, stretched the concurrent attention kernels further; the same 128 waves packed
// into 16 workgroups of 8 staged too slowly).  Lane t takes listing t: a page of a host-pool
// unit is claimed for this call by moving its map entry to the call's epoch (the lane whose
// exchange returns another epoch wins, so each distinct page is claimed once per call), gets the
// next staging slot (or -1 when the pool is full) and publishes it in map_slot.  The wave then
// copies its claimed pages one after another, all 64 lanes moving 16-byte pieces with 8 loads in
// flight each.  The selection call that follows reads map_slot only for entries stamped with its
// own epoch, after this kernel has completed.
struct StageArgs {
  const int32_t* ids;
  int64_t is1, is2, is3;
  const int32_t* unit;
  const unsigned char* host_k;
  const unsigned char* host_v;
  const float* host_sk;
  const float* host_sv;
  unsigned char* stage_k;
  unsigned char* stage_v;
  float* stage_sk;
  float* stage_sv;
  int32_t* map_epoch;
  int32_t* map_slot;
  int32_t* counter;
  int64_t page_bytes;
  int H, T, max_chunks, n_chunks, ppc, n_host, slots, epoch;
};

__device__ __forceinline__ void stage_copy_page(const unsigned char* src, unsigned char* dst,
                                                int64_t bytes, int lane) {
  constexpr int kBatch = 8;
  for (int64_t base = 0; base < bytes; base += static_cast<int64_t>(kBatch) * kWave * 16) {
    uint4 r[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t off = base + static_cast<int64_t>(j * kWave + lane) * 16;
      if (off < bytes) r[j] = *reinterpret_cast<const uint4*>(src + off);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t off = base + static_cast<int64_t>(j * kWave + lane) * 16;
      if (off < bytes) *reinterpret_cast<uint4*>(dst + off) = r[j];
    }
  }
}

constexpr int kStageWaves = 128;

__global__ __launch_bounds__(kWave) void paged_stage_kernel(StageArgs a, int rows) {
  const int lane = lane_id();
  for (int row = static_cast<int>(blockIdx.x); row < rows; row += static_cast<int>(gridDim.x)) {
  const int g = row / a.H, h = row - g * a.H;
  for (int t0 = 0; t0 < a.T; t0 += kWave) {
    const int t = t0 + lane;
    int slot = -1, src_page = 0;
    if (t < a.T) {
      const int32_t bid = a.ids[g * a.is1 + h * a.is2 + t * a.is3];
      if (bid >= 0) {
        const int cid = bid / a.ppc, p = bid - cid * a.ppc;
        if (cid < a.n_chunks && cid < a.max_chunks) {
          const int32_t s = a.unit[static_cast<int64_t>(h) * a.max_chunks + cid];
          if (s <= -2 && -2 - s < a.n_host) {
            const int64_t mi = (static_cast<int64_t>(h) * a.max_chunks + cid) * a.ppc + p;
            if (atomicExch(a.map_epoch + mi, a.epoch) != a.epoch) {
              const int ss = atomicAdd(a.counter, 1);
              slot = ss < a.slots ? ss : -1;
              a.map_slot[mi] = slot;
              src_page = (-2 - s) * a.ppc + p;
            }
          }
        }
      }
    }
    uint64_t m = __ballot(slot >= 0);
    while (m != 0ull) {
      const int l = __builtin_ctzll(m);
      m &= m - 1ull;
      const int ss = __builtin_amdgcn_readlane(slot, l);
      const int sp = __builtin_amdgcn_readlane(src_page, l);
      const int64_t so = static_cast<int64_t>(sp) * a.page_bytes;
      const int64_t dof = static_cast<int64_t>(ss) * a.page_bytes;
      stage_copy_page(a.host_k + so, a.stage_k + dof, a.page_bytes, lane);
      stage_copy_page(a.host_v + so, a.stage_v + dof, a.page_bytes, lane);
      if (a.stage_sk != nullptr && lane == 0) {
        a.stage_sk[ss] = a.host_sk[sp];
        a.stage_sv[ss] = a.host_sv[sp];
      }
    }
  }
  }
}
}  // namespace
}  // namespace omm

extern "C" int omm_paged_stage(const omm_paged_kv* kv, const omm_view4* ids, int32_t epoch,
                               void* stream) {
  using namespace omm;
  OMM_REQUIRE(kv != nullptr && ids != nullptr, OMM_EINVAL, "omm_paged_stage: null argument");
  OMM_REQUIRE(epoch > 0, OMM_EINVAL, "omm_paged_stage: epoch must be positive");
  OMM_REQUIRE(kv->stage_map_epoch != nullptr && kv->stage_map_slot != nullptr &&
                  kv->stage_counter != nullptr && kv->stage_k != nullptr &&
                  kv->stage_v != nullptr && kv->stage_slots >= 0,
              OMM_EINVAL, "omm_paged_stage: the cache has no staging pool");
  OMM_REQUIRE(kv->dtype == OMM_BF16 ||
                  (kv->dtype == OMM_FP8E4M3 && kv->stage_scale_k != nullptr &&
                   kv->stage_scale_v != nullptr && kv->host_scale_k != nullptr &&
                   kv->host_scale_v != nullptr),
              OMM_EINVAL, "omm_paged_stage: cache dtype / scale arrays");
  OMM_REQUIRE(kv->unit_table != nullptr && kv->page_tokens >= 1 &&
                  kv->pages_per_chunk == cdiv64(kv->chunk_len, kv->page_tokens) &&
                  kv->num_heads >= 1 && kv->head_dim >= 1,
              OMM_EINVAL, "omm_paged_stage: inconsistent cache geometry");
  OMM_REQUIRE(ids->size[0] == 1 && ids->size[2] == kv->num_heads && ids->size[3] >= 1 &&
                  ids->size[1] >= 0 && ids->size[1] * kv->num_heads <= 2147483647ll,
              OMM_EINVAL, "omm_paged_stage: ids must be [1, MG, %d, T]", kv->num_heads);
  const int64_t elem = kv->dtype == OMM_BF16 ? 2 : 1;
  const int64_t page_bytes = static_cast<int64_t>(kv->page_tokens) * kv->head_dim * elem;
  OMM_REQUIRE(page_bytes % 16 == 0 &&
                  (reinterpret_cast<uintptr_t>(kv->host_k) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(kv->host_v) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(kv->stage_k) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(kv->stage_v) & 15u) == 0,
              OMM_EUNSUPPORTED, "omm_paged_stage: pages must be whole 16-byte pieces, pools "
              "16-byte aligned");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = fill_i32(kv->stage_counter, 1, 0, s);
  if (rc) return rc;
  const int64_t rows = ids->size[1] * kv->num_heads;
  if (rows == 0 || kv->n_host_slots == 0) return OMM_OK;
  StageArgs a{};
  a.ids = static_cast<const int32_t*>(ids->data);
  a.is1 = ids->stride[1]; a.is2 = ids->stride[2]; a.is3 = ids->stride[3];
  a.unit = kv->unit_table;
  a.host_k = static_cast<const unsigned char*>(kv->host_k);
  a.host_v = static_cast<const unsigned char*>(kv->host_v);
  a.host_sk = kv->host_scale_k; a.host_sv = kv->host_scale_v;
  a.stage_k = static_cast<unsigned char*>(kv->stage_k);
  a.stage_v = static_cast<unsigned char*>(kv->stage_v);
  a.stage_sk = kv->dtype == OMM_BF16 ? nullptr : kv->stage_scale_k;
  a.stage_sv = kv->dtype == OMM_BF16 ? nullptr : kv->stage_scale_v;
  a.map_epoch = kv->stage_map_epoch; a.map_slot = kv->stage_map_slot;
  a.counter = kv->stage_counter;
  a.page_bytes = page_bytes;
  a.H = kv->num_heads; a.T = static_cast<int>(ids->size[3]);
  a.max_chunks = kv->max_chunks; a.n_chunks = kv->n_chunks; a.ppc = kv->pages_per_chunk;
  a.n_host = kv->n_host_slots; a.slots = kv->stage_slots; a.epoch = epoch;
  paged_stage_kernel<<<static_cast<unsigned>(std::min<int64_t>(rows, kStageWaves)), kWave, 0, s>>>(
      a, static_cast<int>(rows));
  return check_launch("omm_paged_stage");
}

extern "C" int omm_copy_units(const void* src_k, void* dst_k, const void* src_v, void* dst_v,
                              const void* src_sk, void* dst_sk, const void* src_sv, void* dst_sv,
                              const int32_t* src_slot, const int32_t* dst_slot, int32_t n,
                              int32_t n_src_slots, int32_t n_dst_slots, int64_t unit_bytes,
                              int64_t scale_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE(n >= 0 && unit_bytes > 0 && unit_bytes % 16 == 0 && scale_bytes >= 0, OMM_EINVAL,
              "omm_copy_units: n >= 0 and unit_bytes a positive multiple of 16 required");
  if (n == 0) return OMM_OK;
  OMM_REQUIRE(src_k && dst_k && src_slot && dst_slot, OMM_EINVAL, "omm_copy_units: null pointer");
  OMM_REQUIRE((src_v == nullptr) == (dst_v == nullptr) && (src_sk == nullptr) == (dst_sk == nullptr) &&
                  (src_sv == nullptr) == (dst_sv == nullptr),
              OMM_EINVAL, "omm_copy_units: source and destination pairs must both be given");
  for (const void* p : {src_k, static_cast<const void*>(dst_k), src_v, static_cast<const void*>(dst_v)})
    OMM_REQUIRE((reinterpret_cast<uintptr_t>(p) & 15u) == 0, OMM_EINVAL,
                "omm_copy_units: pools must be 16-byte aligned");
  CopyArgs a{static_cast<const unsigned char*>(src_k), static_cast<unsigned char*>(dst_k),
             static_cast<const unsigned char*>(src_v), static_cast<unsigned char*>(dst_v),
             static_cast<const unsigned char*>(src_sk), static_cast<unsigned char*>(dst_sk),
             static_cast<const unsigned char*>(src_sv), static_cast<unsigned char*>(dst_sv),
             src_slot, dst_slot, unit_bytes, scale_bytes, n_src_slots, n_dst_slots};
  const dim3 grid(static_cast<unsigned>(n), static_cast<unsigned>(cdiv64(unit_bytes, kCopyPart)));
  copy_units_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return check_launch("omm_copy_units");
}

extern "C" int omm_copy_units_async(const void* src_k, void* dst_k, const void* src_v,
                                    void* dst_v, const void* src_sk, void* dst_sk,
                                    const void* src_sv, void* dst_sv,
                                    const int32_t* src_slot_host, const int32_t* dst_slot_host,
                                    int32_t n, int32_t n_src_slots, int32_t n_dst_slots,
                                    int64_t unit_bytes, int64_t scale_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE(n >= 0 && unit_bytes > 0 && scale_bytes >= 0, OMM_EINVAL,
              "omm_copy_units_async: n >= 0 and unit_bytes > 0 required");
  if (n == 0) return OMM_OK;
  OMM_REQUIRE(src_k && dst_k && src_slot_host && dst_slot_host, OMM_EINVAL,
              "omm_copy_units_async: null pointer");
  OMM_REQUIRE((src_v == nullptr) == (dst_v == nullptr) && (src_sk == nullptr) == (dst_sk == nullptr) &&
                  (src_sv == nullptr) == (dst_sv == nullptr),
              OMM_EINVAL, "omm_copy_units_async: source and destination pairs must both be given");
  for (int32_t i = 0; i < n; ++i)
    OMM_REQUIRE(src_slot_host[i] >= 0 && src_slot_host[i] < n_src_slots &&
                    dst_slot_host[i] >= 0 && dst_slot_host[i] < n_dst_slots,
                OMM_EINVAL, "omm_copy_units_async: slot pair %d (%d -> %d) out of range", i,
                src_slot_host[i], dst_slot_host[i]);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto copy = [&](const void* src, void* dst, int64_t bytes, int64_t a, int64_t b, int64_t cnt) {
    if (src == nullptr || bytes == 0) return hipSuccess;
    return hipMemcpyAsync(static_cast<unsigned char*>(dst) + b * bytes,
                          static_cast<const unsigned char*>(src) + a * bytes, cnt * bytes,
                          hipMemcpyDefault, s);
  };
  for (int32_t i = 0; i < n;) {
    int32_t j = i + 1;  // a run of units consecutive in both pools
    while (j < n && src_slot_host[j] == src_slot_host[j - 1] + 1 &&
           dst_slot_host[j] == dst_slot_host[j - 1] + 1)
      ++j;
    const int64_t a = src_slot_host[i], b = dst_slot_host[i], cnt = j - i;
    for (hipError_t e : {copy(src_k, dst_k, unit_bytes, a, b, cnt),
                         copy(src_v, dst_v, unit_bytes, a, b, cnt),
                         copy(src_sk, dst_sk, scale_bytes, a, b, cnt),
                         copy(src_sv, dst_sv, scale_bytes, a, b, cnt)})
      OMM_REQUIRE(e == hipSuccess, OMM_EHIP, "omm_copy_units_async: %s", hipGetErrorString(e));
    i = j;
  }
  return OMM_OK;
}

extern "C" int omm_gather_publish_clear(const int64_t* desc, int64_t n_fetch, int64_t n_clear,
                                        int64_t block_bytes, int64_t* ctas, void* stream) {
  using namespace omm;
  if (ctas != nullptr) *ctas = 0;
  if (n_fetch == 0 && n_clear == 0) return OMM_OK;
  OMM_REQUIRE(n_fetch >= 0 && n_clear >= 0, OMM_EINVAL,
              "omm_gather_publish_clear: n_fetch=%lld / n_clear=%lld must be >= 0",
              (long long)n_fetch, (long long)n_clear);
  OMM_REQUIRE(desc != nullptr, OMM_EINVAL, "omm_gather_publish_clear: null descriptor");
  OMM_REQUIRE(block_bytes > 0 && block_bytes % 2 == 0, OMM_EINVAL,
              "omm_gather_publish_clear: block_bytes=%lld must be a positive multiple of 2",
              (long long)block_bytes);
  const int64_t wgs = n_fetch + cdiv64(n_clear, kClearPerWg);
  OMM_REQUIRE(wgs <= 2147483647ll, OMM_EUNSUPPORTED, "omm_gather_publish_clear: grid too large");
  gather_publish_clear_kernel<<<static_cast<unsigned>(wgs), 256, 0, static_cast<hipStream_t>(stream)>>>(
      desc, n_fetch, n_clear, block_bytes);
  const int rc = check_launch("omm_gather_publish_clear");
  if (rc == OMM_OK && ctas != nullptr) *ctas = wgs;
  return rc;
}

extern "C" int omm_block_range(int64_t* table, int32_t* n_valid, int64_t heads, int64_t mb,
                               int64_t first_bid, int64_t n_blocks, int64_t k_base,
                               int64_t v_base, int64_t head_stride_bytes, int64_t block_bytes,
                               int64_t n_valid_value, int32_t write_k, int32_t write_v,
                               int32_t clear, void* stream) {
  using namespace omm;
  OMM_REQUIRE(table != nullptr && n_valid != nullptr && heads > 0 && mb > 0, OMM_EINVAL,
              "omm_block_range: null table or empty geometry");
  OMM_REQUIRE(n_blocks > 0 && first_bid >= 0 && first_bid + n_blocks <= mb, OMM_EINVAL,
              "omm_block_range: block range [%lld, %lld) outside [0, %lld)", (long long)first_bid,
              (long long)(first_bid + n_blocks), (long long)mb);
  OMM_REQUIRE(n_valid_value <= 2147483647ll, OMM_EINVAL, "omm_block_range: n_valid_value too large");
  if (!clear) {
    OMM_REQUIRE(write_k || write_v, OMM_EINVAL, "omm_block_range: nothing to register");
    OMM_REQUIRE(!write_k || k_base != 0, OMM_EINVAL, "omm_block_range: write_k with k_base == 0");
    OMM_REQUIRE(!write_v || v_base != 0, OMM_EINVAL, "omm_block_range: write_v with v_base == 0");
  }
  const int64_t tiles = cdiv64(n_blocks, 128);
  OMM_REQUIRE(tiles <= 65535 && heads <= 2147483647ll, OMM_EUNSUPPORTED,
              "omm_block_range: %lld blocks exceed the grid", (long long)n_blocks);
  const dim3 grid(static_cast<unsigned>(heads), static_cast<unsigned>(tiles));
  block_range_kernel<<<grid, 128, 0, static_cast<hipStream_t>(stream)>>>(
      table, n_valid, heads, mb, first_bid, n_blocks, k_base, v_base, head_stride_bytes,
      block_bytes, n_valid_value, write_k != 0, write_v != 0, clear != 0);
  return check_launch("omm_block_range");
}

extern "C" int omm_dedup_run(const int32_t* block_indices, int64_t n_entries, int32_t* stamp,
                             int32_t* counts, int32_t* offsets, int32_t* out, int64_t epoch,
                             int64_t mb, int64_t heads, int64_t t, int64_t bpc, int64_t cap,
                             void* stream) {
  using namespace omm;
  OMM_REQUIRE(mb > 0 && heads > 0 && t > 0 && bpc > 0 && mb % bpc == 0, OMM_EINVAL,
              "omm_dedup_run: need positive mb/heads/t/bpc with bpc | mb (mb=%lld heads=%lld t=%lld "
              "bpc=%lld)", (long long)mb, (long long)heads, (long long)t, (long long)bpc);
  const int64_t n_keys = heads * mb;
  OMM_REQUIRE(n_keys <= 2147483647ll, OMM_EINVAL, "omm_dedup_run: %lld keys do not fit int32",
              (long long)n_keys);
  const int64_t n_tiles = cdiv64(n_keys, kDedupTile);
  OMM_REQUIRE(n_tiles <= kDedupMaxTiles, OMM_EUNSUPPORTED, "omm_dedup_run: %lld tiles", (long long)n_tiles);
  OMM_REQUIRE(epoch >= 1 && epoch <= 2147483647ll && cap >= 0, OMM_EINVAL,
              "omm_dedup_run: epoch must be in [1, INT32_MAX] and cap >= 0");
  OMM_REQUIRE(n_entries >= 0 && n_entries <= 2147483647ll, OMM_EINVAL,
              "omm_dedup_run: n_entries out of range");
  OMM_REQUIRE(stamp && counts && offsets && out && (n_entries == 0 || block_indices), OMM_EINVAL,
              "omm_dedup_run: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned mark = static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(cdiv64(n_entries, 256), 1), 8192));
  dedup_mark_kernel<<<mark, 256, 0, s>>>(block_indices, n_entries, stamp, static_cast<int32_t>(epoch),
                                         static_cast<int32_t>(mb), static_cast<int32_t>(heads),
                                         static_cast<int32_t>(t), static_cast<int32_t>(bpc));
  int rc = check_launch("omm_dedup_run mark");
  if (rc) return rc;
  dedup_count_kernel<<<static_cast<unsigned>(n_tiles), kDedupThreads, 0, s>>>(stamp, counts, n_keys,
                                                                              static_cast<int32_t>(epoch));
  rc = check_launch("omm_dedup_run count");
  if (rc) return rc;
  dedup_scan_kernel<<<1, kDedupThreads, 0, s>>>(counts, offsets, out, static_cast<int>(n_tiles));
  rc = check_launch("omm_dedup_run scan");
  if (rc) return rc;
  dedup_compact_kernel<<<static_cast<unsigned>(n_tiles), kDedupThreads, 0, s>>>(
      stamp, offsets, out, n_keys, cap, static_cast<int32_t>(epoch));
  return check_launch("omm_dedup_run compact");
}
