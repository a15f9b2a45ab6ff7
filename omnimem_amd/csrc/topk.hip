// Block scoring + top-k selection.
//
// Reference semantics: cuda_backend/csrc/topk.cu -- visibility rule (:36-97), ordering
// (score desc, id asc; :3, :100-102), -1 padding and output contract (ops.h:11-12).
// Design (gfx950): one workgroup = 8 query rows x one column span of one (b, h).
//   1. scores: the span's compressed keys stream through LDS in 64-column tiles; every thread
//      owns one column and two rows and accumulates fmaf over d in ascending order, so the fp32
//      score is a fixed function of its inputs (reproduced bit-for-bit by the C oracle).
//   2. selection, one wave per row: theta = topk-th largest of the 64 per-lane maxima (one
//      wave-wide bitonic sort); only keys >= theta survive (at most topk lanes contribute);
//      each survivor's exact rank among survivors is counted from LDS; rank < topk is written.
//   Rows whose span is split (long key histories) write packed keys and a merge kernel selects
//   again over the per-span winners.
#include "omm_common.h"

namespace omm {
namespace {

constexpr int kRG = 8;            // query rows per workgroup
constexpr int kThreads = 256;     // 4 waves
constexpr int kTileC = 64;        // key columns per LDS tile
constexpr int kSurvCap = 512;     // survivor slots per wave
constexpr int kMaxSpan = 2048;    // columns per workgroup (score buffer 8 x 2048 fp32)
constexpr int kMaxSplit = 32;

struct MaskDev {
  int bs, G, chunk_q, chunk_k, bpc, qoff, q_half, k_half, ex_win, ex_sink;
  int causal, tf, prog;
};

struct RowInfo {
  int q_cid, q_rel;
  bool q_clean, do_excl;
};

__device__ __forceinline__ RowInfo row_info(const MaskDev& m, int g) {
  RowInfo r;
  r.q_cid = static_cast<int>((static_cast<int64_t>(g) * m.G) / m.chunk_q) + m.qoff;
  if (m.tf) {
    r.q_clean = r.q_cid < m.q_half;
    r.q_rel = r.q_clean ? r.q_cid : r.q_cid - m.q_half;
  } else {
    r.q_clean = true;
    r.q_rel = r.q_cid;
  }
  r.do_excl = m.prog ? (r.q_rel >= m.ex_sink + m.ex_win) : true;
  return r;
}

__device__ __forceinline__ int col_cid(const MaskDev& m, int c) {
  return m.bpc > 0 ? c / m.bpc : static_cast<int>((static_cast<int64_t>(c) * m.bs) / m.chunk_k);
}

__device__ __forceinline__ bool visible(const MaskDev& m, const RowInfo& r, int k_cid) {
  const bool k_clean = m.tf ? (k_cid < m.k_half) : true;
  const int k_rel = (m.tf && !k_clean) ? (k_cid - m.k_half) : k_cid;
  bool ok;
  if (m.tf) {
    ok = (r.q_clean && k_clean && k_rel <= r.q_rel) ||     // clean -> clean, causal
         (!r.q_clean && k_clean && k_rel < r.q_rel) ||     // noisy -> earlier clean
         (!r.q_clean && !k_clean && k_rel == r.q_rel);     // noisy -> own noisy chunk
  } else {
    ok = m.causal ? (k_cid <= r.q_cid) : true;
  }
  if (m.ex_sink > 0) {
    const bool past_sink = !k_clean || k_rel >= m.ex_sink;
    ok = ok && (past_sink || !r.do_excl);
  }
  if (m.ex_win > 0) {
    bool in_win;
    if (m.tf) {
      in_win = k_clean && k_rel >= r.q_rel - m.ex_win + 1;
    } else {
      in_win = k_cid >= r.q_cid - m.ex_win + 1;
      if (!m.causal) in_win = in_win && k_cid <= r.q_cid + m.ex_win - 1;
    }
    ok = ok && (!in_win || !r.do_excl);
  }
  return ok;
}

// Exclusive bound on the visible columns of a row (chunk-causal / tf bound only).
__device__ __forceinline__ int row_ub(const MaskDev& m, const RowInfo& r, int NC) {
  int chunk_ub;
  if (m.tf) {
    chunk_ub = r.q_clean ? r.q_rel + 1 : m.k_half + r.q_rel + 1;
  } else if (m.causal) {
    chunk_ub = r.q_cid + 1;
  } else {
    return NC;
  }
  if (chunk_ub <= 0) return 0;
  const int64_t ub = m.bpc > 0 ? static_cast<int64_t>(chunk_ub) * m.bpc
                               : (static_cast<int64_t>(chunk_ub) * m.chunk_k + m.bs - 1) / m.bs;
  return static_cast<int>(ub < NC ? ub : NC);
}

// ---- selection over n candidates of one row, one wave -------------------------------------
// key(i) gives the packed key of candidate i < n (0 = not a candidate).  emit(rank, key) for
// rank < topk; pad(p) for output positions p >= number of candidates.  All lanes of the wave
// must call this; sv is the wave's LDS survivor buffer.
template <typename KeyF, typename EmitF, typename PadF>
__device__ __forceinline__ void wave_select(int n, int topk, KeyF key, EmitF emit, PadF pad,
                                            uint64_t* sv) {
  const int lane = lane_id();
  const int per = (n + kWave - 1) / kWave;
  uint64_t lmax = 0;
  for (int j = 0; j < per; ++j) {
    const int i = j * kWave + lane;
    if (i < n) {
      const uint64_t k = key(i);
      lmax = k > lmax ? k : lmax;
    }
  }
  const uint64_t sorted = wave_sort_desc(lmax);
  const uint32_t t_lo = __shfl(static_cast<uint32_t>(sorted), topk - 1, kWave);
  const uint32_t t_hi = __shfl(static_cast<uint32_t>(sorted >> 32), topk - 1, kWave);
  const uint64_t theta = (static_cast<uint64_t>(t_hi) << 32) | t_lo;

  int ns = 0;
  for (int j = 0; j < per; ++j) {
    const int i = j * kWave + lane;
    const uint64_t k = (i < n) ? key(i) : 0ull;
    const bool surv = k != 0ull && k >= theta;
    const uint64_t m = ballot64(surv);
    const int pos = ns + lanes_below(m);
    if (surv && pos < kSurvCap) sv[pos] = k;
    ns += popc64(m);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (ns <= kSurvCap) {
    // exact rank of each survivor among the survivors (keys are distinct)
    for (int i = lane; i < ns; i += kWave) {
      const uint64_t k = sv[i];
      int rank = 0;
      for (int j = 0; j < ns; ++j) rank += (sv[j] > k) ? 1 : 0;
      if (rank < topk) emit(rank, k);
    }
  } else {
    // too many survivors for the buffer (scores periodic in the lane stride): extract the
    // maxima one at a time, each a wave-wide max over the keys below the previous one
    uint64_t prev = ~0ull;
    int r = 0;
    for (; r < topk; ++r) {
      uint64_t best = 0;
      for (int j = 0; j < per; ++j) {
        const int i = j * kWave + lane;
        const uint64_t k = (i < n) ? key(i) : 0ull;
        if (k < prev && k > best) best = k;
      }
#pragma unroll
      for (int mm = 1; mm < kWave; mm <<= 1) {
        const uint64_t o = shfl_xor_u64(best, mm);
        best = o > best ? o : best;
      }
      if (best == 0ull) break;
      if (lane == 0) emit(r, best);
      prev = best;
    }
    ns = r;
  }
  for (int p = lane; p < topk; p += kWave)
    if (p >= ns) pad(p);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 8 consecutive T from LDS as floats (p 16-byte aligned).
template <typename T> __device__ __forceinline__ void lds8(const T* p, float (&f)[8]);
template <> __device__ __forceinline__ void lds8<bf16_t>(const bf16_t* p, float (&f)[8]) {
  const uint4 r = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void lds8<f16_t>(const f16_t* p, float (&f)[8]) {
  const uint4 r = *reinterpret_cast<const uint4*>(p);
  const f16_t* e = reinterpret_cast<const f16_t*>(&r);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = static_cast<float>(e[i].v);
}
template <> __device__ __forceinline__ void lds8<float>(const float* p, float (&f)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

template <typename T> __host__ __device__ constexpr int kpad() { return 16 / static_cast<int>(sizeof(T)); }

// Dynamic LDS: sc [kRG][span] f32 | sv [4][kSurvCap] u64 | qs [kRG][DP] f32 | ks [64][DP+pad] T
template <typename T, bool FROM_SCORES>
__global__ __launch_bounds__(kThreads) void topk_kernel(
    View4<const T> q, View4<const T> k, const float* __restrict__ scores, int MG, int H, int D,
    int NC, int topk, float scale, MaskDev mk, int span, int nsplit, int32_t* __restrict__ out,
    uint64_t* __restrict__ part) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int bh = blockIdx.z, b = bh / H, h = bh - b * H;
  const int row0 = blockIdx.x * kRG, split = blockIdx.y;

  int ub = 0;
#pragma unroll
  for (int r = 0; r < kRG; ++r) {
    const int g = row0 + r;
    if (g < MG) ub = max(ub, row_ub(mk, row_info(mk, g), NC));
  }
  const int c_begin = split * span;
  const int c_end = min(c_begin + span, ub);
  const int n = max(0, c_end - c_begin);

  float* sc = reinterpret_cast<float*>(smem);
  uint64_t* sv = reinterpret_cast<uint64_t*>(smem + static_cast<size_t>(kRG) * span * 4);

  if constexpr (!FROM_SCORES) {
    const int DP = (D + 7) & ~7;
    const int KP = DP + kpad<T>();
    float* qs = reinterpret_cast<float*>(sv + 4 * kSurvCap);
    T* ks = reinterpret_cast<T*>(qs + kRG * DP);
    for (int i = tid; i < kRG * DP; i += kThreads) {
      const int r = i / DP, d = i - r * DP, g = row0 + r;
      qs[i] = (g < MG && d < D) ? to_f32<T>(*q.at(b, g, h, d)) : 0.0f;
    }
    const int c = tid & (kTileC - 1), rp = tid / kTileC;  // rows 2rp, 2rp+1
    for (int c0 = c_begin; c0 < c_end; c0 += kTileC) {
      __syncthreads();
      for (int i = tid; i < kTileC * DP; i += kThreads) {
        const int cc = i / DP, d = i - cc * DP, col = c0 + cc;
        ks[cc * KP + d] = (col < c_end && d < D) ? *k.at(b, col, h, d) : from_f32<T>(0.0f);
      }
      __syncthreads();
      const T* kr = ks + c * KP;
      const float* q0 = qs + (2 * rp) * DP;
      const float* q1 = q0 + DP;
      float a0 = 0.0f, a1 = 0.0f;
      for (int d = 0; d < DP; d += 8) {
        float kv[8], x0[8], x1[8];
        lds8<T>(kr + d, kv);
        lds8<float>(q0 + d, x0);
        lds8<float>(q1 + d, x1);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          a0 = __builtin_fmaf(x0[u], kv[u], a0);
          a1 = __builtin_fmaf(x1[u], kv[u], a1);
        }
      }
      if (c0 + c < c_end) {
        sc[(2 * rp) * span + (c0 + c - c_begin)] = a0 * scale;
        sc[(2 * rp + 1) * span + (c0 + c - c_begin)] = a1 * scale;
      }
    }
  } else {
    for (int i = tid; i < kRG * n; i += kThreads) {
      const int r = i / n, j = i - r * n, g = row0 + r;
      sc[r * span + j] =
          (g < MG) ? scores[((static_cast<int64_t>(b) * MG + g) * H + h) * NC + c_begin + j] : 0.0f;
    }
  }
  __syncthreads();

  uint64_t* wsv = sv + wave * kSurvCap;
  for (int rr = 0; rr < kRG / 4; ++rr) {
    const int r = wave + 4 * rr, g = row0 + r;
    if (g >= MG) continue;  // wave-uniform; no workgroup barrier below
    const RowInfo ri = row_info(mk, g);
    const float* srow = sc + r * span;
    const int64_t orow = (static_cast<int64_t>(b) * MG + g) * H + h;
    auto key = [&](int i) -> uint64_t {
      const int col = c_begin + i;
      return visible(mk, ri, col_cid(mk, col)) ? make_key(srow[i], col, NC) : 0ull;
    };
    if (nsplit == 1) {
      int32_t* o = out + orow * topk;
      wave_select(n, topk, key, [&](int rank, uint64_t kk) { o[rank] = key_id(kk, NC); },
                  [&](int p) { o[p] = -1; }, wsv);
    } else {
      uint64_t* o = part + (orow * nsplit + split) * topk;
      wave_select(n, topk, key, [&](int rank, uint64_t kk) { o[rank] = kk; },
                  [&](int p) { o[p] = 0ull; }, wsv);
    }
    (void)lane;
  }
}

// One wave per row: top-k over the nsplit * topk per-span winners.
__global__ __launch_bounds__(kThreads) void topk_merge_kernel(const uint64_t* __restrict__ part,
                                                              int32_t* __restrict__ out,
                                                              int64_t rows, int nsplit, int topk,
                                                              int NC) {
  __shared__ uint64_t sv[4 * kSurvCap];
  const int wave = threadIdx.x / kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (row >= rows) return;  // wave-uniform; no workgroup barrier in this kernel
  const uint64_t* p = part + row * nsplit * topk;
  int32_t* o = out + row * topk;
  wave_select(
      nsplit * topk, topk, [&](int i) { return p[i]; },
      [&](int rank, uint64_t kk) { o[rank] = key_id(kk, NC); }, [&](int q) { o[q] = -1; },
      sv + wave * kSurvCap);
}

struct Plan {
  int span, nsplit;
  size_t ws;
};

Plan make_plan(int64_t B, int64_t MG, int64_t H, int64_t NC, int topk) {
  Plan p{};
  const int span_max = kMaxSpan;
  int nsplit = static_cast<int>(cdiv64(NC, span_max));
  if (nsplit < 1) nsplit = 1;
  // spread long rows over more workgroups when there are few rows
  const int64_t tiles = cdiv64(MG, kRG) * B * H;
  const int64_t want = 512;
  if (tiles * nsplit < want) {
    const int64_t extra = cdiv64(want, tiles);
    const int64_t by_len = cdiv64(NC, 256);
    int64_t ns = std::min<int64_t>(extra, by_len);
    if (ns > nsplit) nsplit = static_cast<int>(ns);
  }
  nsplit = std::min(nsplit, kMaxSplit);
  int span = static_cast<int>(cdiv64(NC, nsplit));
  span = (span + kTileC - 1) & ~(kTileC - 1);
  if (span < kTileC) span = kTileC;
  p.span = span;
  p.nsplit = nsplit;
  p.ws = nsplit > 1 ? static_cast<size_t>(B * MG * H) * nsplit * topk * sizeof(uint64_t) : 0;
  return p;
}

int check_mask(const omm_topk_mask* m) {
  OMM_REQUIRE(m != nullptr, OMM_EINVAL, "top-k: null mask");
  OMM_REQUIRE(m->block_size > 0 && m->group_size > 0 && m->chunk_q > 0 && m->chunk_k > 0,
              OMM_EINVAL, "top-k: block_size / group_size / chunk_q / chunk_k must be > 0");
  OMM_REQUIRE(m->blocks_per_chunk >= 0 && m->q_chunk_offset >= 0 && m->ex_win >= 0 &&
                  m->ex_sink >= 0 && m->q_half >= 0 && m->k_half >= 0,
              OMM_EINVAL, "top-k: negative mask parameter");
  OMM_REQUIRE(!(m->tf_mask && m->q_chunk_offset != 0), OMM_EINVAL,
              "top-k: tf_mask assumes a full [clean|noisy] layout, q_chunk_offset must be 0");
  return OMM_OK;
}

MaskDev to_dev(const omm_topk_mask& m) {
  return MaskDev{m.block_size, m.group_size, m.chunk_q, m.chunk_k, m.blocks_per_chunk,
                 m.q_chunk_offset, m.q_half, m.k_half, m.ex_win, m.ex_sink,
                 m.causal != 0, m.tf_mask != 0, m.prog_excl != 0};
}

template <typename T, bool FS>
int launch_topk(const omm_view4* q, const omm_view4* k, const float* scores, int64_t B,
                int64_t MG, int64_t H, int64_t NC, int D, int topk, float scale,
                const omm_topk_mask& mask, int32_t* out, void* ws, size_t ws_bytes,
                hipStream_t stream) {
  const Plan p = make_plan(B, MG, H, NC, topk);
  OMM_REQUIRE(p.ws <= ws_bytes && (p.ws == 0 || ws != nullptr), OMM_EWORKSPACE,
              "top-k: workspace of %zu bytes required, got %zu", p.ws, ws_bytes);
  size_t smem = static_cast<size_t>(kRG) * p.span * 4 + 4 * kSurvCap * sizeof(uint64_t);
  if (!FS) {
    const int DP = (D + 7) & ~7;
    smem += static_cast<size_t>(kRG) * DP * 4 + static_cast<size_t>(kTileC) * (DP + kpad<T>()) * sizeof(T);
  }
  OMM_REQUIRE(smem <= 160 * 1024, OMM_EUNSUPPORTED, "top-k: %zu bytes of LDS needed", smem);
  if (smem > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_kernel<T, FS>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(smem));
    if (e != hipSuccess) return set_error(OMM_EHIP, "top-k: LDS attribute: %s", hipGetErrorString(e));
  }
  const dim3 grid(static_cast<unsigned>(cdiv64(MG, kRG)), static_cast<unsigned>(p.nsplit),
                  static_cast<unsigned>(B * H));
  View4<const T> qv{}, kv{};
  if (!FS) {
    qv = make_view<const T>(*q);
    kv = make_view<const T>(*k);
  }
  uint64_t* part = static_cast<uint64_t*>(ws);
  topk_kernel<T, FS><<<grid, kThreads, smem, stream>>>(qv, kv, scores, static_cast<int>(MG),
                                         static_cast<int>(H), D, static_cast<int>(NC), topk,
                                         scale, to_dev(mask), p.span, p.nsplit, out, part);
  int rc = check_launch("top-k");
  if (rc != OMM_OK || p.nsplit == 1) return rc;
  const int64_t rows = B * MG * H;
  topk_merge_kernel<<<static_cast<unsigned>(cdiv64(rows, 4)), kThreads, 0, stream>>>(
      part, out, rows, p.nsplit, topk, static_cast<int>(NC));
  return check_launch("top-k merge");
}

int check_sizes(int64_t B, int64_t MG, int64_t H, int64_t NC, int32_t topk) {
  OMM_REQUIRE(B >= 0 && MG >= 0 && H >= 0 && NC >= 0, OMM_EINVAL, "top-k: negative size");
  OMM_REQUIRE(topk >= 1 && topk <= 64, OMM_EUNSUPPORTED, "top-k: topk must be in [1, 64], got %d",
              topk);
  OMM_REQUIRE(B * H <= 65535 && cdiv64(MG, kRG) <= 2147483647ll, OMM_EUNSUPPORTED,
              "top-k: B*H must be <= 65535");
  OMM_REQUIRE(NC <= static_cast<int64_t>(kMaxSpan) * kMaxSplit, OMM_EUNSUPPORTED,
              "top-k: %lld key blocks exceed the supported %lld", (long long)NC,
              (long long)kMaxSpan * kMaxSplit);
  return OMM_OK;
}

}  // namespace
}  // namespace omm

extern "C" size_t omm_topk_workspace_bytes(int64_t B, int64_t MG, int64_t H, int64_t NC,
                                           int32_t topk) {
  if (B <= 0 || MG <= 0 || H <= 0 || NC <= 0 || topk < 1 || topk > 64) return 0;
  return omm::make_plan(B, MG, H, NC, topk).ws;
}

extern "C" int omm_topk(const omm_view4* q, const omm_view4* k, int32_t dtype, int32_t topk,
                        float scale, const omm_topk_mask* mask, int32_t* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE(q != nullptr && k != nullptr && out != nullptr, OMM_EINVAL, "omm_topk: null argument");
  int rc = check_mask(mask);
  if (rc) return rc;
  const int64_t B = q->size[0], MG = q->size[1], H = q->size[2], D = q->size[3], NC = k->size[1];
  OMM_REQUIRE(k->size[0] == B && k->size[2] == H && k->size[3] == D, OMM_EINVAL,
              "omm_topk: incompatible q [%lld,%lld,%lld,%lld] and k [%lld,%lld,%lld,%lld]",
              (long long)B, (long long)MG, (long long)H, (long long)D, (long long)k->size[0],
              (long long)k->size[1], (long long)k->size[2], (long long)k->size[3]);
  OMM_REQUIRE(D >= 1 && D <= 256, OMM_EUNSUPPORTED, "omm_topk: head dim must be in [1, 256], got %lld",
              (long long)D);
  rc = check_sizes(B, MG, H, NC, topk);
  if (rc) return rc;
  if (B == 0 || MG == 0 || H == 0) return OMM_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (NC == 0) {
    return fill_i32(out, B * MG * H * topk, -1, s);
  }
  switch (dtype) {
    case OMM_F32:
      return launch_topk<float, false>(q, k, nullptr, B, MG, H, NC, static_cast<int>(D), topk, scale,
                                       *mask, out, workspace, workspace_bytes, s);
    case OMM_BF16:
      return launch_topk<bf16_t, false>(q, k, nullptr, B, MG, H, NC, static_cast<int>(D), topk,
                                        scale, *mask, out, workspace, workspace_bytes, s);
    case OMM_F16:
      return launch_topk<f16_t, false>(q, k, nullptr, B, MG, H, NC, static_cast<int>(D), topk,
                                       scale, *mask, out, workspace, workspace_bytes, s);
    default: return set_error(OMM_EINVAL, "omm_topk: unsupported dtype %d", dtype);
  }
}

extern "C" int omm_topk_from_scores(const float* scores, int64_t B, int64_t MG, int64_t H,
                                    int64_t NC, int32_t topk, const omm_topk_mask* mask,
                                    int32_t* out, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  using namespace omm;
  OMM_REQUIRE(out != nullptr, OMM_EINVAL, "omm_topk_from_scores: null output");
  int rc = check_mask(mask);
  if (rc) return rc;
  rc = check_sizes(B, MG, H, NC, topk);
  if (rc) return rc;
  if (B == 0 || MG == 0 || H == 0) return OMM_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (NC == 0) {
    return fill_i32(out, B * MG * H * topk, -1, s);
  }
  OMM_REQUIRE(scores != nullptr, OMM_EINVAL, "omm_topk_from_scores: null scores");
  return launch_topk<float, true>(nullptr, nullptr, scores, B, MG, H, NC, 0, topk, 0.0f, *mask, out,
                                  workspace, workspace_bytes, s);
}
