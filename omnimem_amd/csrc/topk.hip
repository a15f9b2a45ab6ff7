// Block scoring + top-k selection.
//
// Reference semantics: cuda_backend/csrc/topk.cu -- visibility rule (:36-97), ordering
// (score desc, id asc; :3, :100-102), -1 padding and output contract (ops.h:11-12).
//
// gfx950 design: one workgroup = 12 query rows x one column span of one (b, h), 4 waves.  Two
// workgroups fit a CU; 12 rows rather than 16 put the 6144 rows of a 32768-token, 12-head call
// (64-token groups) on 516 workgroups, about two per CU, instead of 384 (one CU in two holding
// two while the others held one).
//   1. rows: pooled query rows are staged in LDS as fp32.  In the fused mode the workgroup
//      pools them itself from the full-resolution queries (16-byte loads, fp32 sum in ascending
//      token order, one division, one rounding to the element type -- the omm_block_pool
//      arithmetic), so q is read from HBM exactly once.
//   2. scores: compressed keys stream through LDS in 64-column tiles (16-byte loads, the next
//      tile's loads in flight during the current tile's arithmetic); lane = column, each wave
//      owns 4 rows, and every score is fmaf over d ascending from 0, then * scale, so the fp32
//      score is a fixed function of its inputs (reproduced bit for bit by the C oracle).
//   3. selection, one wave per row: keys in registers; theta = topk-th largest score word of the
//      64 per-lane maxima (ranked across lanes), past topk 64 the exact topk-th largest score
//      word (wave radix select); only keys at or above it survive;
//      each survivor's exact rank among survivors is counted from LDS; rank < topk is written.
//      Column chunk ids are precomputed once per workgroup in LDS.
//   Rows whose columns are split over several workgroups (long key histories) write packed
//   keys and a merge kernel selects again over the per-span winners.
// topk > 128 (the reference's path B): the same scoring writes every row's scores to the
// workspace and topk_large_kernel selects per row (radix select, then an LDS bitonic sort).
#include "omm_common.h"

#include <mutex>
#include <type_traits>

namespace omm {
namespace {

constexpr int kRG = 12;                 // query rows per workgroup (3 per wave)
constexpr int kThreads = 256;           // 4 waves
constexpr int kWaves = kThreads / kWave;
constexpr int kRowsPerWave = kRG / kWaves;
constexpr int kTileC = 64;              // key columns per LDS tile
constexpr int kSurvCap = 256;           // survivor slots per wave
static_assert(kSurvCap % 64 == 0, "survivors are ranked 8 at a time, a wave's 64 lanes each");
constexpr int kSpanCap = 1024;          // columns per workgroup
constexpr int kMaxSplit = 64;
constexpr int kMaxTopk = 128;           // the reference's path A bound (topk.cu:584, 648-660)
constexpr size_t kLdsBudget = 80 * 1024;  // two workgroups per CU
constexpr int kStageRegs = 8;           // 16-byte staging registers per thread (K tile)

enum { kModePooled = 0, kModeFused = 1, kModeScores = 2 };

struct MaskDev {
  int bs, G, chunk_q, chunk_k, bpc, qoff, q_half, k_half, ex_win, ex_sink;
  int causal, tf, prog;
};

struct RowInfo {
  int q_cid, q_rel;
  bool q_clean, do_excl;
};

// num / den for num >= 0, den >= 1: 32-bit division when num fits (the usual case)
__device__ __forceinline__ int64_t div_nn(int64_t num, int den) {
  if (num <= 0xffffffffll)
    return static_cast<int64_t>(static_cast<uint32_t>(num) / static_cast<uint32_t>(den));
  return num / den;
}

__device__ __forceinline__ RowInfo row_info(const MaskDev& m, int g) {
  RowInfo r;
  r.q_cid = static_cast<int>(div_nn(static_cast<int64_t>(g) * m.G, m.chunk_q)) + m.qoff;
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
// key(i) gives the packed key of candidate i < n (0 = not a candidate).
// emit(rank, key) for rank < topk; pad(p) for output positions p >= number of candidates.  All
// lanes of the wave must call this; sv is the wave's LDS survivor buffer.
//   1. every lane loads its keys (candidates lane, lane + 64, ...) into registers once;
//   2. theta = the topk-th largest high word (score half) of the 64 per-lane maxima, from each
//      lane's rank among them (readlane compares, no LDS and no scalar round trips);
//   3. survivors = keys whose high word is >= theta (at least topk of them whenever that many
//      candidates exist, and every key of the top topk), compacted into sv;
//   4. each survivor's exact rank among the survivors (keys are distinct) -> emit if < topk.
constexpr int kMaxPer = kSpanCap / kWave;

// Wave-wide max of an unsigned value (DPP row shifts and row broadcasts; every lane gets it).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_max(uint32_t v) {
  const uint32_t t = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
  return v > t ? v : t;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = dpp_max<0x111, 0xf>(v);  // row_shr:1
  v = dpp_max<0x112, 0xf>(v);  // row_shr:2
  v = dpp_max<0x114, 0xf>(v);  // row_shr:4
  v = dpp_max<0x118, 0xf>(v);  // row_shr:8 -> lane 15 of each row holds the row max
  v = dpp_max<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  v = dpp_max<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3 -> lane 63 holds the wave max
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), kWave - 1));
}

// The topk-th largest of the 64 lane values v (0 if topk > 64): every lane counts the values
// >= its own (64 LDS broadcast values in the wave-private scratch), and the answer is the
// largest value whose count reaches topk.  scratch: 64 words of wave-private LDS.
__device__ __forceinline__ uint32_t lane_max_threshold(uint32_t v, int topk, uint32_t* scratch) {
  if (topk > kWave) return 0u;
  const int lane = lane_id();
  scratch[lane] = v;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kWave / 4; ++j) {
    const uint4 w = reinterpret_cast<const uint4*>(scratch)[j];
    cnt += (w.x >= v ? 1 : 0) + (w.y >= v ? 1 : 0) + (w.z >= v ? 1 : 0) + (w.w >= v ? 1 : 0);
  }
  const uint32_t theta = wave_max_u32(cnt >= topk ? v : 0u);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // scratch is reused after this
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return theta;
}

// For 64 < topk <= 128: the exact topk-th largest high word among the wave's candidates, by a
// radix select over the 32-bit high words (4 passes of 8 bits, each a 256-bin histogram in the
// wave's LDS scratch and a scan of the bins from the top), so that about topk keys survive.  1
// when fewer than topk candidates exist (every candidate passes: candidates have a high word
// >= 1).  hi(j, ok) gives the high word of the lane's j-th key (j < nper) and whether it is a
// candidate.  scratch: 256 words of wave-private LDS.
template <typename HiF>
__device__ __forceinline__ uint32_t wave_radix_threshold(int nper, int topk, HiF hi,
                                                         uint32_t* scratch) {
  const int lane = lane_id();
  uint32_t prefix = 0u, pmask = 0u;
  uint32_t need = static_cast<uint32_t>(topk);
  for (int shift = 24; shift >= 0; shift -= 8) {
#pragma unroll
    for (int j = 0; j < 256 / kWave; ++j) scratch[lane + kWave * j] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int j = 0; j < nper; ++j) {
      bool ok;
      const uint32_t h = hi(j, ok);
      if (ok && (h & pmask) == prefix) atomicAdd(&scratch[(h >> shift) & 255u], 1u);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // lane l holds bins 255 - 4 l .. 252 - 4 l; running counts from the top bin down
    uint32_t hb[4], sum = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      hb[j] = scratch[255 - 4 * lane - j];
      sum += hb[j];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), d, kWave));
      if (lane >= d) incl += o;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // scratch is rewritten next
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), kWave - 1));
    if (shift == 24 && total < need) return 1u;  // wave-uniform
    uint32_t acc = incl - sum;
    const bool cross = acc < need && incl >= need;  // exactly one lane
    int bin = 0;
    uint32_t above = 0u;
    if (cross) {
      for (int j = 0; j < 4; ++j) {
        if (acc + hb[j] >= need) {
          bin = 255 - 4 * lane - j;
          above = acc;
          break;
        }
        acc += hb[j];
      }
    }
    const int cl = __builtin_ctzll(ballot64(cross));
    bin = __builtin_amdgcn_readlane(bin, cl);
    above = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(above), cl));
    prefix |= static_cast<uint32_t>(bin) << shift;
    pmask |= 255u << shift;
    need -= above;
  }
  return prefix;
}

template <int PER, typename KeyF, typename EmitF, typename PadF>
__device__ __forceinline__ void wave_select_impl(int n, int topk, KeyF key, EmitF emit, PadF pad,
                                                 uint64_t* sv) {
  const int lane = lane_id();
  // keys of slots j * 64 + lane; slots past n read candidate n - 1 (in bounds) and count as 0
  uint64_t kv[PER];
  uint32_t lmax = 0;  // high word of the lane's largest key
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = j * kWave + lane;
    const uint64_t k = key(i < n ? i : n - 1);
    kv[j] = i < n ? k : 0ull;
    const uint32_t h = static_cast<uint32_t>(kv[j] >> 32);
    lmax = h > lmax ? h : lmax;
  }
  // theta: the topk-th largest lane maximum (0 if fewer than topk lanes hold candidates); past
  // 64, the exact topk-th largest high word
  const uint32_t theta = topk <= kWave
      ? lane_max_threshold(lmax, topk, reinterpret_cast<uint32_t*>(sv))
      : wave_radix_threshold(
            PER, topk,
            [&](int j, bool& ok) {
              ok = kv[j] != 0ull;
              return static_cast<uint32_t>(kv[j] >> 32);
            },
            reinterpret_cast<uint32_t*>(sv));

  int ns = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint64_t k = kv[j];
    const bool surv = k != 0ull && static_cast<uint32_t>(k >> 32) >= theta;
    const uint64_t m = ballot64(surv);
    const int pos = ns + lanes_below(m);
    if (surv && pos < kSurvCap) sv[pos] = k;
    ns += popc64(m);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (ns <= kWave) {
    // one survivor per lane; survivors past ns read as 0 (below every key), so groups of 8
    // broadcast reads need no bound checks
    const uint64_t mine = lane < ns ? sv[lane] : 0ull;
    if (lane >= ns && lane < ((ns + 7) & ~7)) sv[lane] = 0ull;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int rank = 0;
    for (int j = 0; j < ns; j += 8) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const ulonglong2 w = reinterpret_cast<const ulonglong2*>(sv + j)[e];
        rank += (w.x > mine ? 1 : 0) + (w.y > mine ? 1 : 0);
      }
    }
    if (lane < ns && rank < topk) emit(rank, mine);
  } else if (ns <= kSurvCap) {
    // lane ranks survivors lane, lane + 64, ... against all of them, 8 broadcast keys a round
    // for all of its survivors at once; slots from ns up to the next multiple of 8 read as 0
    constexpr int MS = kSurvCap / kWave;
    uint64_t mine[MS];
    int rank[MS];
#pragma unroll
    for (int m = 0; m < MS; ++m) {
      const int i = lane + kWave * m;
      mine[m] = i < ns ? sv[i] : 0ull;
      rank[m] = 0;
    }
    if (lane < ((ns + 7) & ~7) - ns) sv[ns + lane] = 0ull;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int j = 0; j < ns; j += 8) {
      ulonglong2 w8[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) w8[q] = reinterpret_cast<const ulonglong2*>(sv + j)[q];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int m = 0; m < MS; ++m)
          rank[m] += (w8[q].x > mine[m] ? 1 : 0) + (w8[q].y > mine[m] ? 1 : 0);
    }
#pragma unroll
    for (int m = 0; m < MS; ++m)
      if (lane + kWave * m < ns && rank[m] < topk) emit(rank[m], mine[m]);
  } else {
    // too many survivors for the buffer (massive score ties): extract the maxima one at a
    // time, each a wave-wide max over the keys below the previous one
    uint64_t prev = ~0ull;
    int r = 0;
    for (; r < topk; ++r) {
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const uint64_t k = kv[j];
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

// Any n (the merge of many column spans): keys are re-read per pass instead of held.
template <typename KeyF, typename EmitF, typename PadF>
__device__ __forceinline__ void wave_select_stream(int n, int topk, KeyF key, EmitF emit,
                                                   PadF pad, uint64_t* sv) {
  const int lane = lane_id();
  const int per = (n + kWave - 1) / kWave;
  uint32_t lmax = 0;
  for (int j = 0; j < per; ++j) {
    const int i = j * kWave + lane;
    if (i < n) {
      const uint32_t h = static_cast<uint32_t>(key(i) >> 32);
      lmax = h > lmax ? h : lmax;
    }
  }
  const uint32_t theta = topk <= kWave
      ? lane_max_threshold(lmax, topk, reinterpret_cast<uint32_t*>(sv))
      : wave_radix_threshold(
            per, topk,
            [&](int j, bool& ok) {
              const int i = j * kWave + lane;
              const uint64_t k = i < n ? key(i) : 0ull;
              ok = k != 0ull;
              return static_cast<uint32_t>(k >> 32);
            },
            reinterpret_cast<uint32_t*>(sv));
  int ns = 0;
  for (int j = 0; j < per; ++j) {
    const int i = j * kWave + lane;
    const uint64_t k = (i < n) ? key(i) : 0ull;
    const bool surv = k != 0ull && static_cast<uint32_t>(k >> 32) >= theta;
    const uint64_t m = ballot64(surv);
    const int pos = ns + lanes_below(m);
    if (surv && pos < kSurvCap) sv[pos] = k;
    ns += popc64(m);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (ns <= kSurvCap) {
    for (int i = lane; i < ns; i += kWave) {
      const uint64_t k = sv[i];
      int rank = 0;
      for (int j = 0; j < ns; ++j) rank += (sv[j] > k) ? 1 : 0;
      if (rank < topk) emit(rank, k);
    }
  } else {
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

template <typename KeyF, typename EmitF, typename PadF>
__device__ __forceinline__ void wave_select(int n, int topk, KeyF key, EmitF emit, PadF pad,
                                            uint64_t* sv) {
  if (n <= 0) {  // no candidates (wave-uniform): all padding
    for (int p = lane_id(); p < topk; p += kWave) pad(p);
    return;
  }
  if (n > kMaxPer * kWave) {
    wave_select_stream(n, topk, key, emit, pad, sv);
    return;
  }
  if (n <= 4 * kWave)
    wave_select_impl<4>(n, topk, key, emit, pad, sv);
  else if (n <= 8 * kWave)
    wave_select_impl<8>(n, topk, key, emit, pad, sv);
  else
    wave_select_impl<kMaxPer>(n, topk, key, emit, pad, sv);
}

// ---- element helpers ------------------------------------------------------------------------
template <typename T> struct Pk { static constexpr int V = 16 / static_cast<int>(sizeof(T)); };

// The V elements of a 16-byte register group as floats.
template <typename T> __device__ __forceinline__ void unpack(const uint4& r, float* f);
template <> __device__ __forceinline__ void unpack<bf16_t>(const uint4& r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack<f16_t>(const uint4& r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i])));
    f[2 * i + 1] =
        static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[i] >> 16)));
  }
}
template <> __device__ __forceinline__ void unpack<float>(const uint4& r, float* f) {
  f[0] = __builtin_bit_cast(float, r.x);
  f[1] = __builtin_bit_cast(float, r.y);
  f[2] = __builtin_bit_cast(float, r.z);
  f[3] = __builtin_bit_cast(float, r.w);
}

// 8 consecutive elements from LDS as floats (p 16-byte aligned).
template <typename T> __device__ __forceinline__ void lds8(const T* p, float (&f)[8]) {
  if constexpr (Pk<T>::V == 8) {
    unpack<T>(*reinterpret_cast<const uint4*>(p), f);
  } else {
    unpack<T>(*reinterpret_cast<const uint4*>(p), f);
    unpack<T>(*reinterpret_cast<const uint4*>(p + 4), f + 4);
  }
}
__device__ __forceinline__ void lds8f(const float* p, float (&f)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

__host__ __device__ constexpr int round8(int d) { return (d + 7) & ~7; }
template <typename T> __host__ __device__ constexpr int kpitch(int D) {
  return round8(D) + Pk<T>::V;  // one 16-byte pad per key row
}

struct Lds {
  size_t sc, sv, kc, qs, ks, total;
};

__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~static_cast<size_t>(15); }

inline Lds lds_layout(int span, int D, int esize, bool scores) {
  Lds l{};
  size_t off = 0;
  l.sc = off; off = align16(off + static_cast<size_t>(kRG) * span * 4);
  l.sv = off; off = align16(off + static_cast<size_t>(kWaves) * kSurvCap * 8);
  l.kc = off; off = align16(off + static_cast<size_t>(span) * 4);
  l.qs = off;
  if (!scores) {
    off = align16(off + static_cast<size_t>(kRG) * round8(D) * 4);
    l.ks = off;
    off = align16(off + static_cast<size_t>(kTileC) * (round8(D) + 16 / esize) * esize);
  }
  l.total = off;
  return l;
}

// Argument block (passed by value; offsets in bytes into dynamic LDS).
struct TopkArgs {
  const void* q;       // pooled rows [B, MG, H, D] or full-resolution tokens [B, T, H, D]
  int64_t qs0, qs1, qs2, qs3;
  const void* k;       // [B, NC, H, D]
  int64_t ks0, ks1, ks2, ks3;
  const float* scores; // [B, MG, H, NC] (scores mode)
  int T_len, G;        // fused mode: tokens and tokens per row
  int MG, H, D, NC, topk;
  float scale;
  MaskDev mk;
  int span, nsplit;
  int vec;             // 16-byte loads allowed for q and k
  int32_t* out;
  uint64_t* part;
  float* dump;         // set: write the scores to [B, MG, H, NC] and select nothing
  uint32_t o_sv, o_kc, o_qs, o_ks;
};

template <typename T, int MODE>
__global__ __launch_bounds__(kThreads) void topk_kernel(TopkArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int V = Pk<T>::V;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
  const int bh = blockIdx.z, b = bh / a.H, h = bh - b * a.H;
  // heavy (late, causal) row tiles first
  const int row0 = (static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x)) * kRG;
  const int split = blockIdx.y;
  const MaskDev& mk = a.mk;

  int ub = 0;
#pragma unroll
  for (int r = 0; r < kRG; ++r) {
    const int g = row0 + r;
    if (g < a.MG) ub = max(ub, row_ub(mk, row_info(mk, g), a.NC));
  }
  const int c_begin = split * a.span;
  const int c_end = min(c_begin + a.span, ub);
  const int n = max(0, c_end - c_begin);
  const int span = a.span;

  float* sc = reinterpret_cast<float*>(smem);
  uint64_t* sv = reinterpret_cast<uint64_t*>(smem + a.o_sv);
  int* kc = reinterpret_cast<int*>(smem + a.o_kc);
  for (int i = tid; i < n; i += kThreads) kc[i] = col_cid(mk, c_begin + i);

  if constexpr (MODE != kModeScores) {
    const int D = a.D, DP = round8(D), KP = kpitch<T>(D);
    float* qs = reinterpret_cast<float*>(smem + a.o_qs);
    T* ks = reinterpret_cast<T*>(smem + a.o_ks);
    const T* qp = static_cast<const T*>(a.q);
    const T* kp = static_cast<const T*>(a.k);

    // ---- 1. query rows -> LDS (fp32) ----
    if (tid / 16 < kRG) {  // 16 threads per row
      const int r = tid / 16, p = tid % 16, g = row0 + r;
      float* qrow = qs + r * DP;
      if (a.vec) {
        const int U = D / V;
        for (int u = p; u < U; u += 16) {
          float acc[V];
#pragma unroll
          for (int i = 0; i < V; ++i) acc[i] = 0.0f;
          if (g < a.MG) {
            if constexpr (MODE == kModeFused) {
              const int t0 = g * a.G, t1 = min(t0 + a.G, a.T_len);
              const T* base = qp + b * a.qs0 + h * a.qs2 + u * V;
              int t = t0;
              for (; t + 8 <= t1; t += 8) {
                uint4 rr[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                  rr[j] = *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(t + j) * a.qs1);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                  float f[V];
                  unpack<T>(rr[j], f);
#pragma unroll
                  for (int i = 0; i < V; ++i) acc[i] += f[i];
                }
              }
              for (; t < t1; ++t) {
                const uint4 rr = *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(t) * a.qs1);
                float f[V];
                unpack<T>(rr, f);
#pragma unroll
                for (int i = 0; i < V; ++i) acc[i] += f[i];
              }
              const float cnt = static_cast<float>(t1 - t0);
#pragma unroll
              for (int i = 0; i < V; ++i) acc[i] = to_f32<T>(from_f32<T>(acc[i] / cnt));
            } else {
              const uint4 rr = *reinterpret_cast<const uint4*>(qp + b * a.qs0 + g * a.qs1 + h * a.qs2 + u * V);
              unpack<T>(rr, acc);
            }
          }
#pragma unroll
          for (int i = 0; i < V; ++i) qrow[u * V + i] = acc[i];
        }
      } else {
        for (int d = p; d < DP; d += 16) {
          float x = 0.0f;
          if (g < a.MG && d < D) {
            if constexpr (MODE == kModeFused) {
              const int t0 = g * a.G, t1 = min(t0 + a.G, a.T_len);
              float acc = 0.0f;
              for (int t = t0; t < t1; ++t)
                acc += to_f32<T>(qp[b * a.qs0 + static_cast<int64_t>(t) * a.qs1 + h * a.qs2 + d * a.qs3]);
              x = to_f32<T>(from_f32<T>(acc / static_cast<float>(t1 - t0)));
            } else {
              x = to_f32<T>(qp[b * a.qs0 + g * a.qs1 + h * a.qs2 + d * a.qs3]);
            }
          }
          qrow[d] = x;
        }
      }
    }

    // ---- 2. scores ----
    // K tile staging: unit = 16 bytes; unit u of the tile is column u / U, part u % U
    const int U = DP / V;
    const int units = kTileC * U;
    uint4 st[kStageRegs];
    auto load_tile = [&](int c0) {
#pragma unroll
      for (int j = 0; j < kStageRegs; ++j) {
        const int u = tid + j * kThreads;
        st[j] = make_uint4(0, 0, 0, 0);
        if (u < units) {
          const int cc = u / U, pp = u - cc * U, col = c0 + cc;
          if (col < c_end)
            st[j] = *reinterpret_cast<const uint4*>(kp + b * a.ks0 + static_cast<int64_t>(col) * a.ks1 +
                                                    h * a.ks2 + pp * V);
        }
      }
    };
    auto store_tile = [&]() {
#pragma unroll
      for (int j = 0; j < kStageRegs; ++j) {
        const int u = tid + j * kThreads;
        if (u < units) {
          const int cc = u / U, pp = u - cc * U;
          *reinterpret_cast<uint4*>(ks + cc * KP + pp * V) = st[j];
        }
      }
    };
    if (a.vec && n > 0) load_tile(c_begin);
    for (int c0 = c_begin; c0 < c_end; c0 += kTileC) {
      __syncthreads();
      if (a.vec) {
        store_tile();
      } else {
        for (int i = tid; i < kTileC * DP; i += kThreads) {
          const int cc = i / DP, d = i - cc * DP, col = c0 + cc;
          ks[cc * KP + d] = (col < c_end && d < D)
                                ? kp[b * a.ks0 + static_cast<int64_t>(col) * a.ks1 + h * a.ks2 + d * a.ks3]
                                : from_f32<T>(0.0f);
        }
      }
      __syncthreads();
      if (a.vec && c0 + kTileC < c_end) load_tile(c0 + kTileC);  // in flight during the FMAs
      const T* kr = ks + lane * KP;
      const float* q0 = qs + (wave * kRowsPerWave) * DP;
      float acc[kRowsPerWave];
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) acc[r] = 0.0f;
      for (int d = 0; d < DP; d += 8) {
        float kv[8];
        lds8<T>(kr + d, kv);
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
          float x[8];
          lds8f(q0 + r * DP + d, x);
#pragma unroll
          for (int u = 0; u < 8; ++u) acc[r] = __builtin_fmaf(x[u], kv[u], acc[r]);
        }
      }
      const int col = c0 + lane;
      if (col < c_end) {
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r)
          sc[(wave * kRowsPerWave + r) * span + (col - c_begin)] = acc[r] * a.scale;
      }
    }
  } else {
    for (int i = tid; i < kRG * n; i += kThreads) {
      const int r = i / n, j = i - r * n, g = row0 + r;
      sc[r * span + j] = (g < a.MG)
          ? a.scores[((static_cast<int64_t>(b) * a.MG + g) * a.H + h) * a.NC + c_begin + j]
          : 0.0f;
    }
  }
  __syncthreads();
  if (a.dump != nullptr) {  // scoring only (topk > kMaxTopk): the selection runs per row after
    for (int i = tid; i < kRG * n; i += kThreads) {
      const int r = i / n, j = i - r * n, g = row0 + r;
      if (g < a.MG)
        a.dump[((static_cast<int64_t>(b) * a.MG + g) * a.H + h) * a.NC + c_begin + j] =
            sc[r * span + j];
    }
    return;
  }

  // ---- 3. selection: wave w owns rows w, w + 4, w + 8 ----
  uint64_t* wsv = sv + wave * kSurvCap;
  for (int rr = 0; rr < kRowsPerWave; ++rr) {
    const int r = wave + kWaves * rr, g = row0 + r;
    if (g >= a.MG) continue;  // wave-uniform; no workgroup barrier below
    const RowInfo ri = row_info(mk, g);
    const float* srow = sc + r * span;
    const int64_t orow = (static_cast<int64_t>(b) * a.MG + g) * a.H + h;
    const int NC = a.NC;
    // plain causal / non-causal masks (no tf, no exclusions): the visible columns are exactly
    // those below the row bound, because chunk ids do not decrease with the column
    const bool simple = !mk.tf && mk.ex_sink <= 0 && mk.ex_win <= 0;
    const int rub = row_ub(mk, ri, NC) - c_begin;
    auto key = [&](int i) -> uint64_t {
      const bool vis = simple ? (i < rub) : visible(mk, ri, kc[i]);
      return vis ? make_key(srow[i], c_begin + i, NC) : 0ull;
    };
    if (a.nsplit == 1) {
      int32_t* o = a.out + orow * a.topk;
      wave_select(n, a.topk, key, [&](int rank, uint64_t kk) { o[rank] = key_id(kk, NC); },
                  [&](int p) { o[p] = -1; }, wsv);
    } else {
      uint64_t* o = a.part + (orow * a.nsplit + split) * a.topk;
      wave_select(n, a.topk, key, [&](int rank, uint64_t kk) { o[rank] = kk; },
                  [&](int p) { o[p] = 0ull; }, wsv);
    }
  }
  (void)lane;
}

// One wave per row: top-k over the nsplit * topk per-span winners.
__global__ __launch_bounds__(kThreads) void topk_merge_kernel(const uint64_t* __restrict__ part,
                                                              int32_t* __restrict__ out,
                                                              int64_t rows, int nsplit, int topk,
                                                              int NC) {
  __shared__ uint64_t sv[kWaves * kSurvCap];
  const int wave = threadIdx.x / kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (row >= rows) return;  // wave-uniform; no workgroup barrier in this kernel
  const uint64_t* p = part + row * nsplit * topk;
  int32_t* o = out + row * topk;
  wave_select(
      nsplit * topk, topk, [&](int i) { return p[i]; },
      [&](int rank, uint64_t kk) { o[rank] = key_id(kk, NC); }, [&](int q) { o[q] = -1; },
      sv + wave * kSurvCap);
}

// ---- topk > 128: the reference's path B -----------------------------------------------------
// Past 128 the reference sorts every column of a row (topk.cu:741-807): key f32_to_ord(score)
// for a visible column and 0 for a hidden one, whose value is -1 (topk.cu:163-166, 549-559);
// a stable descending segmented radix sort, so equal keys keep ascending column order; then
// the first topk values, -1 past NC (topk.cu:563-581).  The key is the raw order code, unlike the
// topk <= 128 rule: +0 ranks above -0, and visible -inf and NaN scores are ranked too (a NaN with
// the sign bit clear above every number, one with it set below -inf; the all-ones pattern has
// code 0, level with the hidden columns).
// One workgroup per row: the topk-th largest code by a 4-pass radix select (256-bin LDS
// histograms over the row's codes), then the codes above it and the first codes equal to it in
// column order, sorted in LDS by a bitonic network; their columns are written in that order.
constexpr int kLargeTopkCap = 4096;
constexpr int kLargeThreads = 256;

__device__ __forceinline__ uint32_t f32_ord_raw(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// scores: [rows, NC] fp32 with rows = (b, g, h) in [B, MG, H] order (only the visible columns
// are read); out: [rows, topk].
__global__ __launch_bounds__(kLargeThreads) void topk_large_kernel(const float* __restrict__ scores,
                                                                   int MG, int H, int NC,
                                                                   int topk, MaskDev mk,
                                                                   int32_t* __restrict__ out) {
  __shared__ uint64_t keys[kLargeTopkCap];
  __shared__ uint32_t hist[256];
  __shared__ int sel[2];  // the chosen bin and the count in the bins above it
  __shared__ int wcnt[kLargeThreads / kWave];
  const int tid = static_cast<int>(threadIdx.x), lane = lane_id(), w = tid / kWave;
  const int64_t row = blockIdx.x;
  const int g = static_cast<int>((row / H) % MG);
  const float* srow = scores + row * NC;
  const RowInfo ri = row_info(mk, g);
  const bool simple = !mk.tf && mk.ex_sink <= 0 && mk.ex_win <= 0;
  const int rub = row_ub(mk, ri, NC);
  auto vis = [&](int c) { return c < rub && (simple || visible(mk, ri, col_cid(mk, c))); };
  auto code = [&](int c) -> uint32_t { return vis(c) ? f32_ord_raw(srow[c]) : 0u; };
  const int K = min(topk, NC);

  // radix select, 8 bits a pass from the top: theta = the K-th largest code, `need` = how many
  // codes equal to theta the first K take
  uint32_t prefix = 0u, pmask = 0u;
  int need = K;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0u;  // kLargeThreads == 256 bins
    __syncthreads();
    for (int c = tid; c < NC; c += kLargeThreads) {
      const uint32_t o = code(c);
      if ((o & pmask) == prefix) atomicAdd(&hist[(o >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (w == 0) {
      // lane l holds bins 255 - 4 l .. 252 - 4 l; running counts from the top bin down
      uint32_t hb[4], sum = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hb[j] = hist[255 - 4 * lane - j];
        sum += hb[j];
      }
      uint32_t incl = sum;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), d, kWave));
        if (lane >= d) incl += o;
      }
      uint32_t acc = incl - sum;
      const uint32_t nd = static_cast<uint32_t>(need);
      if (acc < nd && incl >= nd) {  // exactly one lane: the counts reach need inside its bins
        for (int j = 0; j < 4; ++j) {
          if (acc + hb[j] >= nd) {
            sel[0] = 255 - 4 * lane - j;
            sel[1] = static_cast<int>(acc);
            break;
          }
          acc += hb[j];
        }
      }
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(sel[0]) << shift;
    pmask |= 255u << shift;
    need -= sel[1];
    __syncthreads();  // sel and hist are rewritten by the next pass
  }
  const uint32_t theta = prefix;
  const int n_gt = K - need;  // codes above theta, all taken

  // codes above theta in any order (sorted below), then the first `need` equal to it in column
  // order; keys are code << 32 | (NC - 1 - column), so a larger key comes first
  if (tid == 0) sel[0] = 0;
  __syncthreads();
  for (int c = tid; c < NC; c += kLargeThreads) {
    const uint32_t o = code(c);
    if (o > theta) {
      const int slot = atomicAdd(&sel[0], 1);
      keys[slot] = (static_cast<uint64_t>(o) << 32) | static_cast<uint32_t>(NC - 1 - c);
    }
  }
  int base = 0;  // equal codes in earlier rounds (the same in every thread)
  for (int c0 = 0; c0 < NC && base < need; c0 += kLargeThreads) {
    const int c = c0 + tid;
    const bool eq = c < NC && code(c) == theta;
    const uint64_t m = ballot64(eq);
    if (lane == 0) wcnt[w] = popc64(m);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int j = 0; j < kLargeThreads / kWave; ++j) {
      before += j < w ? wcnt[j] : 0;
      total += wcnt[j];
    }
    const int pos = base + before + lanes_below(m);
    if (eq && pos < need)
      keys[n_gt + pos] = (static_cast<uint64_t>(theta) << 32) | static_cast<uint32_t>(NC - 1 - c);
    base += total;
    __syncthreads();  // wcnt is rewritten by the next round
  }

  // bitonic sort of the K keys, descending; the padding keys (0) sort last, and a real key 0
  // equals them bit for bit
  int P = 1;
  while (P < K) P <<= 1;
  for (int i = K + tid; i < P; i += kLargeThreads) keys[i] = 0ull;
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P / 2; i += kLargeThreads) {
        const int x = 2 * i - (i & (stride - 1)), y = x + stride;
        const uint64_t kx = keys[x], ky = keys[y];
        const bool desc = (x & size) == 0;
        if (desc ? (kx < ky) : (kx > ky)) {
          keys[x] = ky;
          keys[y] = kx;
        }
      }
      __syncthreads();
    }
  }
  int32_t* o = out + row * topk;
  for (int p = tid; p < topk; p += kLargeThreads) {
    int v = -1;
    if (p < K) {
      const int c = NC - 1 - static_cast<int>(static_cast<uint32_t>(keys[p]));
      v = vis(c) ? c : -1;
    }
    o[p] = v;
  }
}

// ---- MFMA scoring path ------------------------------------------------------------------------
// bf16 / f16 queries and keys with head dim 64 or 128, unit dim strides and 16-byte aligned
// rows.  Scores are MFMA dot products: each bf16 (f16) product is exact in fp32 and
// v_mfma_f32_16x16x32 sums them in fp32 over d in 32-wide steps, ascending; the sum is then
// multiplied by scale.  That is the role of the reference's TF32 WMMA scoring
// (topk.cu:179-291, an fp32 sum of exact products in the hardware's order); the selection over
// the scores follows the (score desc, id asc) rule bit for bit.
//
// One item = 16 query rows of one (b, h) x one column span, 4 waves:
//   1. rows -> LDS: pooled from the full-resolution queries (fused mode; each lane sums one
//      16-byte slice of one row over its tokens in ascending order, one division, one rounding:
//      the omm_block_pool arithmetic) or loaded as given (pooled mode);
//   2. S^T = K Qp^T: each wave takes 16-column blocks, K fragments straight from global memory
//      (no LDS staging), Qp^T fragments held in registers; scores * scale -> LDS;
//   3. selection, four rows per wave (one per 16-lane DPP row): a row threshold from the lanes'
//      two largest candidates, then the survivors are compacted and ranked exactly.
typedef float m2_f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 m2_bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 m2_f16x8;

template <typename T> struct M2Mfma;
template <> struct M2Mfma<bf16_t> {
  __device__ __forceinline__ static m2_f32x4 run(uint4 a, uint4 b, m2_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(m2_bf16x8, a),
                                                   __builtin_bit_cast(m2_bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct M2Mfma<f16_t> {
  __device__ __forceinline__ static m2_f32x4 run(uint4 a, uint4 b, m2_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(m2_f16x8, a),
                                                  __builtin_bit_cast(m2_f16x8, b), c, 0, 0, 0);
  }
};

constexpr int kM2Rows = 16;
constexpr int kM2Threads = 256;
constexpr int kM2Waves = kM2Threads / kWave;
constexpr int kM2SpanCap = 768;   // columns per item (12 steps of 64 per selecting lane)
constexpr int kM2Batch = 4;       // 16-column blocks whose K fragments are loaded together

struct M2Args {
  const void* q;       // full-resolution [B, T, H, D] (fused) or pooled rows [B, MG, H, D]
  int64_t qs0, qs1, qs2;
  const void* k;       // [B, NC, H, D]
  int64_t ks0, ks1, ks2;
  int T_len, G;        // fused mode: tokens, tokens per row
  int MG, H, NC, topk;
  float scale;
  MaskDev mk;
  int span, nspan, rtiles;
  int32_t* out;        // nspan == 1
  uint64_t* part;      // nspan > 1: [B*MG*H][nspan][topk] packed keys
  float* dump;         // optional: the scores, [B, MG, H, NC]
  uint32_t o_qs, o_sv, o_tv;
};

// Column steps of 64 a selecting lane holds (template instances: 4, 8 or 12 for spans up to
// 256, 512 or 768), and the LDS row pitch of the scores: those whole steps (the selection reads
// 64 j + 4 l + e for j < JM) plus 4 floats, which keeps rows 16-byte aligned and off one
// another's banks.
__host__ __device__ inline int m2_jm(int span) { return span <= 256 ? 4 : span <= 512 ? 8 : 12; }
__host__ __device__ inline int m2_pitch(int span) { return 64 * m2_jm(span) + 4; }

inline size_t m2_lds_bytes(int span, int D) {
  return static_cast<size_t>(kM2Rows) * m2_pitch(span) * 4         // scores
         + static_cast<size_t>(kM2Rows) * (D + 8) * 2              // rows (16-bit)
         + static_cast<size_t>(kM2Waves) * kSurvCap * 8            // survivors
         + static_cast<size_t>(kM2Rows) * 32 * 4;                  // row thresholds
}

// Threshold of a wave's keys for a top-k: lanes in groups of gs consecutive lanes, 64 / gs >=
// topk groups; theta = the smallest non-empty group maximum (high word) when at least topk
// groups are non-empty -- each such group holds a key >= theta, so at least topk keys pass --
// else 1 (every candidate passes: candidates have a high word >= 1).
__device__ __forceinline__ uint32_t group_threshold(uint32_t lmax, int topk) {
  const int lane = lane_id();
  int gs = kWave;
  while (gs > 1 && kWave / gs < topk) gs >>= 1;
  uint32_t gmax = lmax;
  for (int m = 1; m < gs; m <<= 1) {
    const uint32_t o = static_cast<uint32_t>(__shfl_xor(static_cast<int>(gmax), m, kWave));
    gmax = o > gmax ? o : gmax;
  }
  const int groups = popc64(ballot64((lane % gs) == 0 && gmax != 0u));
  uint32_t gmin = gmax != 0u ? gmax : 0xffffffffu;
  for (int m = gs; m < kWave; m <<= 1) {
    const uint32_t o = static_cast<uint32_t>(__shfl_xor(static_cast<int>(gmin), m, kWave));
    gmin = o < gmin ? o : gmin;
  }
  return groups >= topk ? gmin : 1u;
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Top-k of one row from its fp32 scores in LDS (srow[i], i < n = column c_begin + i), one
// wave.  vis(i) says whether column i is visible; -inf and NaN are never candidates.  Keys are
// make_key(score, column): larger = (score desc, id asc).
//   1. lane maxima of the candidates' high words (columns lane, lane + 64, ...) ->
//      theta = group_threshold; candidates >= theta are compacted into sv (LDS, wave-private);
//   2. while more than 64 survive: the survivors (<= 4 per lane) are cut by group_threshold
//      again;
//   3. one survivor per lane is ranked exactly by broadcast reads of the others.
// Ties so massive that a cut removes nothing fall back to taking maxima one at a time.
template <typename VisF, typename EmitF, typename PadF>
__device__ __forceinline__ void row_topk_lds(const float* srow, int n, int c_begin, int NC,
                                             int topk, VisF vis, EmitF emit, PadF pad,
                                             uint64_t* sv) {
  const int lane = lane_id();
  uint32_t lmax = 0;
  for (int i = lane; i < n; i += kWave) {
    const float x = srow[i];
    if (x > kNegInf && vis(i)) {
      const uint32_t hi = f32_ord(x);
      lmax = hi > lmax ? hi : lmax;
    }
  }
  uint32_t theta = group_threshold(lmax, topk);
  int ns = 0;
  for (int i0 = 0; i0 < n; i0 += kWave) {
    const int i = i0 + lane;
    uint64_t k = 0ull;
    if (i < n) {
      const float x = srow[i];
      if (x > kNegInf && f32_ord(x) >= theta && vis(i)) k = make_key(x, c_begin + i, NC);
    }
    const uint64_t m = ballot64(k != 0ull);
    const int pos = ns + lanes_below(m);
    if (k != 0ull && pos < kSurvCap) sv[pos] = k;
    ns += popc64(m);
  }
  wave_lds_sync();
  bool exhaustive = ns > kSurvCap;
  while (!exhaustive && ns > kWave) {
    uint64_t s4[kSurvCap / kWave];
    uint32_t smax = 0;
#pragma unroll
    for (int j = 0; j < kSurvCap / kWave; ++j) {
      const int i = kWave * j + lane;
      s4[j] = i < ns ? sv[i] : 0ull;
      const uint32_t hi = static_cast<uint32_t>(s4[j] >> 32);
      smax = hi > smax ? hi : smax;
    }
    theta = group_threshold(smax, topk);
    wave_lds_sync();  // every lane has read sv
    int ns2 = 0;
#pragma unroll
    for (int j = 0; j < kSurvCap / kWave; ++j) {
      const uint64_t k = s4[j];
      const bool surv = static_cast<uint32_t>(k >> 32) >= theta && k != 0ull;
      const uint64_t m = ballot64(surv);
      if (surv) sv[ns2 + lanes_below(m)] = k;
      ns2 += popc64(m);
    }
    wave_lds_sync();
    if (ns2 == ns) exhaustive = true;  // no progress: ties
    ns = ns2;
  }
  if (!exhaustive) {
    const uint64_t mine = lane < ns ? sv[lane] : 0ull;
    if (lane >= ns && lane < ((ns + 7) & ~7)) sv[lane] = 0ull;  // groups of 8 read below
    wave_lds_sync();
    int rank = 0;
    for (int j = 0; j < ns; j += 8) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const ulonglong2 w = reinterpret_cast<const ulonglong2*>(sv + j)[e];
        rank += (w.x > mine ? 1 : 0) + (w.y > mine ? 1 : 0);
      }
    }
    if (lane < ns && rank < topk) emit(rank, mine);
  } else {
    // the maxima one at a time: each round a wave-wide max over the keys below the previous
    uint64_t prev = ~0ull;
    int r = 0;
    for (; r < topk; ++r) {
      uint64_t best = 0ull;
      for (int i = lane; i < n; i += kWave) {
        const float x = srow[i];
        if (x > kNegInf && vis(i)) {
          const uint64_t k = make_key(x, c_begin + i, NC);
          if (k < prev && k > best) best = k;
        }
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
  wave_lds_sync();
}

// ---- four rows per wave, one row per 16-lane DPP row (topk <= 16) ----------------------------
// DPP reductions inside a 16-lane row: every lane gets the row's maximum / the inclusive prefix.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
  v = max(v, dpp_u32<0x121>(v));  // row_ror:1
  v = max(v, dpp_u32<0x122>(v));  // row_ror:2
  v = max(v, dpp_u32<0x124>(v));  // row_ror:4
  v = max(v, dpp_u32<0x128>(v));  // row_ror:8
  return v;
}
// Row maximum of NaN-free floats (-inf the smallest): float max over the rotated copies.
__device__ __forceinline__ float row16_max_f(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  v = fmaxf(v, __builtin_bit_cast(float, dpp_u32<0x121>(b)));
  v = fmaxf(v, __builtin_bit_cast(float, dpp_u32<0x122>(__builtin_bit_cast(uint32_t, v))));
  v = fmaxf(v, __builtin_bit_cast(float, dpp_u32<0x124>(__builtin_bit_cast(uint32_t, v))));
  v = fmaxf(v, __builtin_bit_cast(float, dpp_u32<0x128>(__builtin_bit_cast(uint32_t, v))));
  return v;
}
// inclusive prefix sum over the lanes of a 16-lane row (row_shr with zero fill)
template <int CTRL>
__device__ __forceinline__ int dpp_shr0(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);  // bound_ctrl: 0 past the edge
}
__device__ __forceinline__ int row16_scan(int v) {
  v += dpp_shr0<0x111>(v);  // row_shr:1
  v += dpp_shr0<0x112>(v);  // row_shr:2
  v += dpp_shr0<0x114>(v);  // row_shr:4
  v += dpp_shr0<0x118>(v);  // row_shr:8
  return v;
}
// the four rows' values of a per-row quantity (lanes 0, 16, 32, 48), reduced on the scalar unit
__device__ __forceinline__ int rows4_max(int v) {
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int rows4_min(int v) {
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

constexpr int kRowSurv = kSurvCap / 4;  // survivor slots per row (64)
constexpr float kPosInf = __builtin_huge_valf();

// Visible columns of one row: [lo0, hi0) and [lo1, hi1), disjoint, either possibly empty
// (lo == hi).  Global columns in the row facts, relative to the item's first column in the
// selection.
struct RowCols {
  int lo0, hi0, lo1, hi1;
};

// ceil(num / den) for num >= 0, den >= 1: 32-bit division when num fits (the usual case)
__device__ __forceinline__ int64_t ceil_div_nn(int64_t num, int den) {
  if (num <= 0xffffffffll) {
    const uint32_t n32 = static_cast<uint32_t>(num), d32 = static_cast<uint32_t>(den);
    const uint32_t q = n32 / d32;
    return static_cast<int64_t>(q) + (n32 - q * d32 != 0u ? 1 : 0);
  }
  return (num + den - 1) / den;
}
// First column whose chunk id (col_cid) is >= x, clamped to [0, NC].
__device__ __forceinline__ int chunk_col(const MaskDev& m, int x, int NC) {
  if (x <= 0) return 0;
  const int64_t c = m.bpc > 0 ? static_cast<int64_t>(x) * m.bpc
                              : ceil_div_nn(static_cast<int64_t>(x) * m.chunk_k, m.bs);
  return c < NC ? static_cast<int>(c) : NC;
}
// The visible rule (`visible` above) as at most two intervals of chunk ids, then of columns:
// the base set is a prefix of the clean chunks (tf: up to the row's own chunk, or the one before
// for noisy rows; causal: up to the row's chunk; else all), the sink exclusion raises its start,
// the window exclusion lowers its end, and the second interval is a noisy row's own noisy chunk
// (tf) or the chunks past a non-causal window.
__device__ __forceinline__ RowCols row_cols(const MaskDev& m, const RowInfo& r, int NC) {
  constexpr int kAll = 0x3fffffff;
  int x0 = 0, y0, x1 = 1, y1 = 0;  // inclusive chunk ids; empty when x > y
  if (m.tf) {
    y0 = min(r.q_clean ? r.q_rel : r.q_rel - 1, m.k_half - 1);
    if (!r.q_clean) x1 = y1 = m.k_half + r.q_rel;
  } else {
    y0 = m.causal ? r.q_cid : kAll;
  }
  if (r.do_excl) {
    if (m.ex_sink > 0) x0 = max(x0, m.ex_sink);
    if (m.ex_win > 0) {
      if (!m.tf && !m.causal) {
        x1 = max(x0, r.q_cid + m.ex_win);
        y1 = y0;
      }
      y0 = min(y0, (m.tf ? r.q_rel : r.q_cid) - m.ex_win);
    }
  }
  RowCols c{0, 0, 0, 0};
  if (x0 <= y0) {
    c.lo0 = chunk_col(m, x0, NC);
    c.hi0 = chunk_col(m, y0 + 1, NC);
  }
  if (x1 <= y1 && y1 >= 0) {
    c.lo1 = chunk_col(m, x1, NC);
    c.hi1 = chunk_col(m, y1 + 1, NC);
  }
  if (c.lo0 >= c.hi0) c.lo0 = c.hi0 = 0;
  if (c.lo1 >= c.hi1) c.lo1 = c.hi1 = 0;
  return c;
}
// a row's intervals relative to column c0 and clipped to [0, n)
__device__ __forceinline__ RowCols clip_cols(RowCols c, int c0, int n) {
  RowCols o;
  o.lo0 = min(max(c.lo0 - c0, 0), n);
  o.hi0 = min(max(c.hi0 - c0, 0), n);
  o.lo1 = min(max(c.lo1 - c0, 0), n);
  o.hi1 = min(max(c.hi1 - c0, 0), n);
  if (o.lo0 >= o.hi0) o.lo0 = o.hi0 = 0;
  if (o.lo1 >= o.hi1) o.lo1 = o.hi1 = 0;
  return o;
}
__device__ __forceinline__ bool in_cols(const RowCols& c, int i) {
  return static_cast<uint32_t>(i - c.lo0) < static_cast<uint32_t>(c.hi0 - c.lo0) ||
         static_cast<uint32_t>(i - c.lo1) < static_cast<uint32_t>(c.hi1 - c.lo1);
}

// Top-k (k <= 16) of the four rows r = 4 w + (lane >> 4) of a wave.  Lane (row, l) holds the
// columns 64 j + 4 l + e (j < JM, e < 4) of its row's LDS scores; rows hold n <= 64 JM columns
// at a pitch SP >= 64 JM, so every read stays in its row.  `rc`: the lane's row's visible
// columns, clipped to [0, n).  The cost is VALU issue (a wave64 instruction takes four cycles),
// so the per-column work is kept to a handful of instructions:
//   - 64-column steps that no row of the wave sees are skipped, steps that every row sees in
//     full take no visibility test, and only the steps at interval edges test each column;
//   - each lane keeps the two largest of its candidates (m1 >= m2, the new second largest is the
//     median of m1, m2 and the value); the row threshold theta is the topk-th largest of the
//     row's 32 values m1, m2, which are scores of distinct columns, so at least topk candidates
//     are >= theta and every key of the top topk is;
//   - survivors (>= theta, about 18 for top-16 of random scores) are compacted per row and
//     ranked exactly.  A row with more than 64 (massive ties) is reported in the returned
//     overflow bits (bit per row) for the caller to redo.
template <int JM, typename EmitF, typename PadF>
__device__ __forceinline__ uint32_t rows4_topk(const float* sc, int SP, int c_begin, int NC,
                                               int topk, bool row_live, RowCols rc, EmitF emit,
                                               PadF pad, uint64_t* sv, uint32_t* tv) {
  using Bits = typename std::conditional<(4 * JM <= 32), uint32_t, uint64_t>::type;
  const int lane = lane_id(), rid = lane >> 4, l16 = lane & 15;
  const float* srow = sc + rid * SP;  // caller offsets sc to the wave's first row
  // steps [t_lo, t_hi) touch a visible column of some row; [f_lo, f_hi) are inside every row's
  // first interval (rows past the tile's end constrain neither)
  int f_lo = 0, f_hi = JM, t_lo = JM, t_hi = 0;
  if (row_live) {
    const bool e0 = rc.lo0 < rc.hi0, e1 = rc.lo1 < rc.hi1;
    f_lo = e0 ? (rc.lo0 + 63) >> 6 : JM;
    f_hi = e0 ? rc.hi0 >> 6 : 0;
    if (e0) { t_lo = rc.lo0 >> 6; t_hi = (rc.hi0 + 63) >> 6; }
    if (e1) { t_lo = min(t_lo, rc.lo1 >> 6); t_hi = max(t_hi, (rc.hi1 + 63) >> 6); }
  }
  const int F_lo = rows4_max(f_lo), F_hi = rows4_min(f_hi);
  const int T_lo = rows4_min(t_lo), T_hi = rows4_max(t_hi);
  // every read is issued before any is used
  float4 x4[JM];
#pragma unroll
  for (int j = 0; j < JM; ++j) x4[j] = *reinterpret_cast<const float4*>(srow + kWave * j + 4 * l16);
  // candidates' scores (-inf for invisible columns) and the lane's two largest.  NaN scores
  // stay as they are: v_med3_f32 with a NaN operand returns the minimum of the others, so
  // med3(m1, m2, NaN) = m2 and med3(m1, NaN, +inf) = m1, and NaN >= thr is false below.
  float xv[JM][4];
  float m1 = kNegInf, m2 = kNegInf;
  // +inf the compiler cannot see: med3(m1, x, +inf) would otherwise become a maxnum, which in
  // IEEE mode costs a canonicalising max per operand
  float pinf = kPosInf;
  __asm__("" : "+v"(pinf));
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const float xs[4] = {x4[j].x, x4[j].y, x4[j].z, x4[j].w};
    if (j < T_lo || j >= T_hi) {  // wave-uniform: no row sees this step
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[j][e] = kNegInf;
      continue;
    }
    if (j < F_lo || j >= F_hi) {  // wave-uniform: an interval edge in some row
      __asm__ volatile("" ::: "memory");  // keeps the test off the steps that need none
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xv[j][e] = in_cols(rc, kWave * j + 4 * l16 + e) ? xs[e] : kNegInf;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[j][e] = xs[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m2 = __builtin_amdgcn_fmed3f(m1, m2, xv[j][e]);
      m1 = __builtin_amdgcn_fmed3f(m1, xv[j][e], pinf);
    }
  }
  // theta: the topk-th largest of the row's 32 values m1, m2 (-inf when fewer are finite)
  float* trow = reinterpret_cast<float*>(tv + rid * 32);
  trow[2 * l16] = m1;
  trow[2 * l16 + 1] = m2;
  wave_lds_sync();
  int c1 = 0, c2 = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float4 t4 = reinterpret_cast<const float4*>(trow)[q];
    c1 += (t4.x >= m1) + (t4.y >= m1) + (t4.z >= m1) + (t4.w >= m1);
    c2 += (t4.x >= m2) + (t4.y >= m2) + (t4.z >= m2) + (t4.w >= m2);
  }
  const float theta = row16_max_f(fmaxf(c1 >= topk ? m1 : kNegInf, c2 >= topk ? m2 : kNegInf));
  // x >= thr is "x >= theta and a candidate": with theta = -inf every candidate passes, and
  // -inf / NaN never do
  const float thr = fmaxf(theta, -__FLT_MAX__);
  // survivors, bit 4 j + e: 32-bit words built as w = 2 w + (x >= thr), highest bit first
  uint32_t sw[(JM + 7) / 8];
#pragma unroll
  for (int q = 0; q < (JM + 7) / 8; ++q) {
    uint32_t v = 0u;
#pragma unroll
    for (int t = (4 * JM - 1 < 32 * q + 31 ? 4 * JM - 1 : 32 * q + 31); t >= 32 * q; --t)
      v = v + v + (xv[t >> 2][t & 3] >= thr ? 1u : 0u);
    sw[q] = row_live ? v : 0u;
  }
  Bits sbits = sw[0];
  if constexpr (JM > 8) sbits |= static_cast<Bits>(sw[(JM + 7) / 8 - 1]) << 32;
  const int cnt = __builtin_popcountll(static_cast<uint64_t>(sbits));
  const int incl = row16_scan(cnt);
  int pos = incl - cnt;
  // row totals: lane 15 of each row
  const int t0 = __builtin_amdgcn_readlane(incl, 15), t1 = __builtin_amdgcn_readlane(incl, 31);
  const int t2 = __builtin_amdgcn_readlane(incl, 47), t3 = __builtin_amdgcn_readlane(incl, 63);
  const int ns = rid == 0 ? t0 : rid == 1 ? t1 : rid == 2 ? t2 : t3;
  const int nmax = max(max(t0 > kRowSurv ? 0 : t0, t1 > kRowSurv ? 0 : t1),
                       max(t2 > kRowSurv ? 0 : t2, t3 > kRowSurv ? 0 : t3));
  uint64_t* srv = sv + rid * kRowSurv;
  wave_lds_sync();  // the threshold buffer may be reused by the caller's next rows
  // write the survivors' keys, two per round (a lane holds a handful): re-read their scores
  while (sbits != 0) {
    const int ta = __builtin_ctzll(static_cast<uint64_t>(sbits));
    sbits &= sbits - 1;
    const bool hb = sbits != 0;
    const int tb = hb ? __builtin_ctzll(static_cast<uint64_t>(sbits)) : ta;
    if (hb) sbits &= sbits - 1;
    const int ia = kWave * (ta >> 2) + 4 * l16 + (ta & 3);
    const int ib = kWave * (tb >> 2) + 4 * l16 + (tb & 3);
    const float xa = srow[ia], xb = srow[ib];
    if (pos < kRowSurv) srv[pos] = make_key(xa, c_begin + ia, NC);
    if (hb && pos + 1 < kRowSurv) srv[pos + 1] = make_key(xb, c_begin + ib, NC);
    pos += hb ? 2 : 1;
  }
  // zeros after a row's survivors up to the wave's read bound (groups of 8): 0 outranks nothing
  const int lim8 = (nmax + 7) & ~7;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int p = ns + l16 + 16 * q;
    if (ns <= kRowSurv && p < lim8) srv[p] = 0ull;
  }
  wave_lds_sync();
  const uint32_t over = static_cast<uint32_t>(ns > kRowSurv);
  const int nsr = ns > kRowSurv ? 0 : ns;  // an overflowing row is left to the caller
  const int M = (nmax + 15) / 16;  // survivors per lane to rank (wave-uniform, <= 4)
  // rank: lane takes survivors l16, l16 + 16, l16 + 32, l16 + 48 of its row
  uint64_t mine[4];
  int rank[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    mine[m] = (m < M && 16 * m + l16 < nsr) ? srv[16 * m + l16] : ~0ull;
    rank[m] = 0;
  }
  for (int i0 = 0; i0 < nmax; i0 += 8) {  // wave-uniform
    ulonglong2 w8[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) w8[q] = *reinterpret_cast<const ulonglong2*>(srv + i0 + 2 * q);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m < M) rank[m] += (w8[q].x > mine[m] ? 1 : 0) + (w8[q].y > mine[m] ? 1 : 0);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m)
    if (m < M && 16 * m + l16 < nsr && rank[m] < topk) emit(rid, rank[m], mine[m]);
  if (!over && l16 < topk && l16 >= nsr && row_live) pad(rid, l16);
  wave_lds_sync();
  // overflow bits of the four rows, wave-uniform
  const uint64_t ob = ballot64(over != 0u && l16 == 0);
  return static_cast<uint32_t>((ob & 1ull) | ((ob >> 15) & 2ull) | ((ob >> 30) & 4ull) |
                               ((ob >> 45) & 8ull));
}

// rows4_topk for a score pitch SP = m2_pitch(span): the instance whose JM the pitch was built for
template <typename EmitF, typename PadF>
__device__ __forceinline__ uint32_t rows4_topk_sp(const float* sc, int SP, int c_begin, int NC,
                                                  int topk, bool row_live, RowCols rc,
                                                  EmitF emit, PadF pad, uint64_t* sv,
                                                  uint32_t* tv) {
  if (SP <= 64 * 4 + 4)
    return rows4_topk<4>(sc, SP, c_begin, NC, topk, row_live, rc, emit, pad, sv, tv);
  if (SP <= 64 * 8 + 4)
    return rows4_topk<8>(sc, SP, c_begin, NC, topk, row_live, rc, emit, pad, sv, tv);
  return rows4_topk<12>(sc, SP, c_begin, NC, topk, row_live, rc, emit, pad, sv, tv);
}

// One workgroup per (b, h, column span, 16-row tile):
//   1. the rows' first loads (fused: the first 16 tokens of each query group; else the pooled
//      rows) and this wave's first K fragments are issued before anything else, then the row
//      facts (visible column intervals) are worked out while they are in flight;
//   2. query-group pooling (fp32 sum in token order, one divide, one rounding) -> LDS;
//   3. S^T = K Qp^T on MFMA, K fragments straight from global memory -> scores * scale in LDS;
//   4. selection: wave w owns rows 4 w .. 4 w + 3, one per 16-lane DPP row.
template <typename T, int D, bool FUSED>
__global__ __launch_bounds__(kM2Threads, 2) void topk_mfma_kernel(M2Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int SD = D / 32;      // MFMA k-steps
  constexpr int CH = D / 8;       // 16-byte slices per row
  constexpr int QP = D + 8;       // LDS row pitch of the pooled rows (elements)
  __shared__ RowCols facts[kM2Rows];
  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
  const int l16 = lane & 15, j4 = lane >> 4;
  const int total = static_cast<int>(gridDim.x);
  int it = xcd_remap(static_cast<int>(blockIdx.x), total);
  // item order: (b, h) major, then column span, then row tiles heaviest (latest) first
  const int rt = a.rtiles - 1 - it % a.rtiles; it /= a.rtiles;
  const int sp = it % a.nspan; it /= a.nspan;
  const int h = it % a.H;
  const int b = it / a.H;
  const int row0 = rt * kM2Rows;
  const int SP = m2_pitch(a.span);
  const int c_begin = sp * a.span;

  float* sc = reinterpret_cast<float*>(smem);
  uint16_t* qs = reinterpret_cast<uint16_t*>(smem + a.o_qs);
  uint64_t* sv = reinterpret_cast<uint64_t*>(smem + a.o_sv);

  // ---- 1. first loads ----
  const T* qp = static_cast<const T*>(a.q);
  const int pr = tid / CH, pu = tid - pr * CH, pg = row0 + pr;  // pooling: row, 16-byte slice
  const bool pooler = tid < kM2Rows * CH && pg < a.MG;
  const T* qbase = qp + b * a.qs0 + h * a.qs2 + pu * 8;
  int t0 = 0, t1 = 0;
  uint4 rr[16];
  bool first = false;
  if constexpr (FUSED) {
    t0 = pg * a.G;
    t1 = min(t0 + a.G, a.T_len);
    first = pooler && t0 + 16 <= t1;
    if (first) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        rr[j] = *reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(t0 + j) * a.qs1);
    }
  } else {
    if (pooler) rr[0] = *reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(pg) * a.qs1);
  }
  // this wave's first batch of K fragments (columns clamped in bounds; unused ones are dropped)
  const T* kp = static_cast<const T*>(a.k) + b * a.ks0 + h * a.ks2;
  // a wave's batches are kM2Stride blocks apart.  The first is issued now and is in flight
  // during the pooling; the second (when the span has one) once this thread's query loads are
  // all issued, so that K's L2 traffic does not take miss slots from the HBM-bound pooling but
  // is in flight across the barrier
  constexpr int kM2Stride = kM2Waves * kM2Batch;
  uint4 kf0[kM2Batch][SD], kf1[kM2Batch][SD];
  auto load_k = [&](uint4 (&kf)[kM2Batch][SD], int cb0) {
#pragma unroll
    for (int x = 0; x < kM2Batch; ++x) {
      const int col = min(c_begin + (cb0 + x) * 16 + l16, a.NC - 1);
#pragma unroll
      for (int s = 0; s < SD; ++s)
        kf[x][s] = *reinterpret_cast<const uint4*>(kp + static_cast<int64_t>(col) * a.ks1 +
                                                   32 * s + 8 * j4);
    }
  };
  const bool pre1 = a.span > 16 * kM2Stride;  // wave-uniform
  load_k(kf0, w * kM2Batch);

  // row facts, lane l16 -> row row0 + l16; the tile's column bound by a row maximum
  int ub;
  {
    const int g = row0 + l16;
    RowCols rc{0, 0, 0, 0};
    if (g < a.MG) rc = row_cols(a.mk, row_info(a.mk, g), a.NC);
    if (w == 0 && lane < kM2Rows) facts[lane] = rc;
    ub = static_cast<int>(row16_max(static_cast<uint32_t>(max(rc.hi0, rc.hi1))));
    ub = __builtin_amdgcn_readfirstlane(ub);  // rows 0-15 in every 16-lane row: wave-uniform
  }
  const int c_end = min(c_begin + a.span, ub);
  const int n = max(0, c_end - c_begin);
  const int nblk = (n + 15) / 16;

  // ---- 2. rows -> LDS ----
  if (tid < kM2Rows * CH) {
    uint4 val = make_uint4(0, 0, 0, 0);
    if (pooler) {
      if constexpr (FUSED) {
        constexpr int V = 8;
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
        auto add = [&](const uint4& x) {
          float f[V];
          unpack<T>(x, f);
#pragma unroll
          for (int i = 0; i < V; ++i) acc[i] += f[i];
        };
        int t = t0;
        if (first) {
#pragma unroll
          for (int j = 0; j < 16; ++j) add(rr[j]);
          t += 16;
        }
        for (; t + 16 <= t1; t += 16) {
#pragma unroll
          for (int j = 0; j < 16; ++j)
            rr[j] = *reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(t + j) * a.qs1);
#pragma unroll
          for (int j = 0; j < 16; ++j) add(rr[j]);
        }
        for (; t < t1; ++t) add(*reinterpret_cast<const uint4*>(qbase + static_cast<int64_t>(t) * a.qs1));
        const float cnt = static_cast<float>(t1 - t0);
        uint16_t bits[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const T x = from_f32<T>(acc[i] / cnt);
          bits[i] = __builtin_bit_cast(uint16_t, x);
        }
        val = make_uint4(bits[0] | (static_cast<uint32_t>(bits[1]) << 16),
                         bits[2] | (static_cast<uint32_t>(bits[3]) << 16),
                         bits[4] | (static_cast<uint32_t>(bits[5]) << 16),
                         bits[6] | (static_cast<uint32_t>(bits[7]) << 16));
      } else {
        val = rr[0];
      }
    }
    *reinterpret_cast<uint4*>(qs + pr * QP + pu * 8) = val;
  }
  if (pre1) load_k(kf1, w * kM2Batch + kM2Stride);
  __syncthreads();

  // ---- 3. S^T = K Qp^T on MFMA -> LDS ----
  uint4 qb[SD];
#pragma unroll
  for (int s = 0; s < SD; ++s)
    qb[s] = *reinterpret_cast<const uint4*>(qs + l16 * QP + 32 * s + 8 * j4);
  auto mfma_batch = [&](const uint4 (&kf)[kM2Batch][SD], int cb0) {
#pragma unroll
    for (int x = 0; x < kM2Batch; ++x) {
      if (cb0 + x >= nblk) break;  // wave-uniform
      m2_f32x4 acc = m2_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < SD; ++s) acc = M2Mfma<T>::run(kf[x][s], qb[s], acc);
      // lane holds the scores of row l16, columns (cb0 + x) * 16 + 4 j4 + 0..3 of the span
      const int c = (cb0 + x) * 16 + 4 * j4;
      const float4 v = make_float4(acc[0] * a.scale, acc[1] * a.scale, acc[2] * a.scale,
                                   acc[3] * a.scale);
      *reinterpret_cast<float4*>(sc + l16 * SP + c) = v;
      if (a.dump != nullptr && row0 + l16 < a.MG) {
        float* d = a.dump + ((static_cast<int64_t>(b) * a.MG + row0 + l16) * a.H + h) * a.NC;
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e < n) d[c_begin + c + e] = vv[e];
      }
    }
  };
  for (int cb0 = w * kM2Batch; cb0 < nblk; cb0 += 2 * kM2Stride) {
    if (cb0 != w * kM2Batch) load_k(kf0, cb0);
    mfma_batch(kf0, cb0);
    const int cb1 = cb0 + kM2Stride;
    if (cb1 >= nblk) break;
    if (cb0 != w * kM2Batch || !pre1) load_k(kf1, cb1);
    mfma_batch(kf1, cb1);
  }
  __syncthreads();

  // ---- 4. selection: wave w owns rows 4 w .. 4 w + 3, one per 16-lane DPP row ----
  uint64_t* wsv = sv + w * kSurvCap;
  uint32_t* wtv = reinterpret_cast<uint32_t*>(smem + a.o_tv) + w * 128;
  const int NC = a.NC;
  const int r = 4 * w + (lane >> 4), g = row0 + r;
  const RowCols rc = clip_cols(facts[r], c_begin, n);
  const int64_t orow = (static_cast<int64_t>(b) * a.MG + g) * a.H + h;
  auto emit_at = [&](int64_t orow_, int rank, uint64_t kk) {
    if (a.nspan == 1) a.out[orow_ * a.topk + rank] = key_id(kk, NC);
    else a.part[(orow_ * a.nspan + sp) * a.topk + rank] = kk;
  };
  auto pad_at = [&](int64_t orow_, int p) {
    if (a.nspan == 1) a.out[orow_ * a.topk + p] = -1;
    else a.part[(orow_ * a.nspan + sp) * a.topk + p] = 0ull;
  };
  uint32_t over = rows4_topk_sp(
      sc + 4 * w * SP, SP, c_begin, NC, a.topk, g < a.MG, rc,
      [&](int, int rank, uint64_t kk) { emit_at(orow, rank, kk); },
      [&](int, int p) { pad_at(orow, p); }, wsv, wtv);
  // rows with more than 64 survivors (massive ties): the whole wave redoes them one at a time
  while (over != 0u) {
    const int rr2 = __builtin_ctz(over);
    over &= over - 1u;
    const int r2 = 4 * w + rr2, g2 = row0 + r2;
    const RowCols rc2 = clip_cols(facts[r2], c_begin, n);
    const int64_t orow2 = (static_cast<int64_t>(b) * a.MG + g2) * a.H + h;
    row_topk_lds(sc + r2 * SP, n, c_begin, NC, a.topk, [&](int i) { return in_cols(rc2, i); },
                 [&](int rank, uint64_t kk) { emit_at(orow2, rank, kk); },
                 [&](int p) { pad_at(orow2, p); }, wsv);
  }
}

// ---- host planning ---------------------------------------------------------------------------
int span_cap(int D, int esize, bool scores) {
  for (int s = kSpanCap; s > kTileC; s -= kTileC)
    if (lds_layout(s, D, esize, scores).total <= kLdsBudget) return s;
  return kTileC;
}

struct Plan {
  int span, nsplit;
  size_t ws_part;
};

// fused: one workgroup per row tile (no column split), so q is pooled exactly once
Plan make_plan(int64_t B, int64_t MG, int64_t H, int64_t NC, int topk, int D, int esize,
               bool scores, bool fused) {
  Plan p{};
  const int cap = span_cap(D, esize, scores);
  int nsplit = static_cast<int>(cdiv64(NC, cap));
  if (nsplit < 1) nsplit = 1;
  const int64_t tiles = cdiv64(MG, kRG) * B * H;
  const int64_t want = 1024;  // ~4 per CU (split spans need less LDS); 512 was 15% slower on AR rows
  if (!fused && tiles * nsplit < want) {
    const int64_t ns = std::min<int64_t>(cdiv64(want, tiles), cdiv64(NC, 128));
    if (ns > nsplit) nsplit = static_cast<int>(ns);
  }
  nsplit = std::min(nsplit, kMaxSplit);
  int span = static_cast<int>(cdiv64(NC, nsplit));
  span = (span + kTileC - 1) & ~(kTileC - 1);
  if (span < kTileC) span = kTileC;
  p.span = span;
  p.nsplit = static_cast<int>(cdiv64(NC, span));
  if (p.nsplit < 1) p.nsplit = 1;
  p.ws_part = p.nsplit > 1 ? static_cast<size_t>(B * MG * H) * p.nsplit * topk * sizeof(uint64_t) : 0;
  return p;
}

bool fused_ok(int64_t B, int64_t MG, int64_t H, int64_t NC, int D, int esize) {
  return cdiv64(NC, span_cap(D, esize, false)) == 1 && cdiv64(MG, kRG) * B * H >= 256;
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

inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 16-byte loads are legal for a [B, L, H, D] view: unit dim stride, D % 8 == 0, every row
// start 16-byte aligned, and one key tile's units fit the staging registers.
bool vec_ok(const omm_view4& v, int esize) {
  const int V = 16 / esize;
  const int D = static_cast<int>(v.size[3]);
  return v.stride[3] == 1 && D % 8 == 0 && a16(v.data) && v.stride[0] % V == 0 &&
         v.stride[1] % V == 0 && v.stride[2] % V == 0 &&
         kTileC * (D / V) <= kStageRegs * kThreads;
}

template <typename T, int MODE>
int launch_core(TopkArgs a, int64_t B, int64_t MG, int64_t H, const Plan& p, int D,
                hipStream_t stream) {
  const Lds l = lds_layout(p.span, D, sizeof(T), MODE == kModeScores);
  OMM_REQUIRE(l.total <= 160 * 1024, OMM_EUNSUPPORTED, "top-k: %zu bytes of LDS needed", l.total);
  if (l.total > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_kernel<T, MODE>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(l.total));
    if (e != hipSuccess) return set_error(OMM_EHIP, "top-k: LDS attribute: %s", hipGetErrorString(e));
  }
  a.span = p.span;
  a.nsplit = p.nsplit;
  a.o_sv = static_cast<uint32_t>(l.sv);
  a.o_kc = static_cast<uint32_t>(l.kc);
  a.o_qs = static_cast<uint32_t>(l.qs);
  a.o_ks = static_cast<uint32_t>(l.ks);
  const dim3 grid(static_cast<unsigned>(cdiv64(MG, kRG)), static_cast<unsigned>(p.nsplit),
                  static_cast<unsigned>(B * H));
  topk_kernel<T, MODE><<<grid, kThreads, l.total, stream>>>(a);
  int rc = check_launch("top-k");
  if (rc != OMM_OK || p.nsplit == 1 || a.dump != nullptr) return rc;
  const int64_t rows = B * MG * H;
  topk_merge_kernel<<<static_cast<unsigned>(cdiv64(rows, kWaves)), kThreads, 0, stream>>>(
      a.part, a.out, rows, p.nsplit, a.topk, a.NC);
  return check_launch("top-k merge");
}

template <int MODE>
int launch_typed(int32_t dtype, TopkArgs a, int64_t B, int64_t MG, int64_t H, const Plan& p,
                 int D, hipStream_t s) {
  switch (dtype) {
    case OMM_F32: return launch_core<float, MODE>(a, B, MG, H, p, D, s);
    case OMM_BF16: return launch_core<bf16_t, MODE>(a, B, MG, H, p, D, s);
    case OMM_F16: return launch_core<f16_t, MODE>(a, B, MG, H, p, D, s);
    default: return set_error(OMM_EINVAL, "top-k: unsupported dtype %d", dtype);
  }
}

int esize_of(int32_t dtype) { return dtype == OMM_F32 ? 4 : 2; }

int check_sizes(int64_t B, int64_t MG, int64_t H, int64_t NC, int32_t topk, int D, int esize,
                bool scores) {
  OMM_REQUIRE(B >= 0 && MG >= 0 && H >= 0 && NC >= 0, OMM_EINVAL, "top-k: negative size");
  OMM_REQUIRE(topk >= 1 && topk <= kLargeTopkCap, OMM_EUNSUPPORTED,
              "top-k: topk must be in [1, %d], got %d", kLargeTopkCap, topk);
  OMM_REQUIRE(B * H <= 65535 && cdiv64(MG, kRG) <= 2147483647ll && MG <= 2147483647ll,
              OMM_EUNSUPPORTED, "top-k: B*H must be <= 65535");
  const int64_t cap = static_cast<int64_t>(span_cap(D, esize, scores)) * kMaxSplit;
  OMM_REQUIRE(NC <= cap, OMM_EUNSUPPORTED, "top-k: %lld key blocks exceed the supported %lld",
              (long long)NC, (long long)cap);
  return OMM_OK;
}

TopkArgs base_args(int64_t MG, int64_t H, int64_t NC, int D, int topk, float scale,
                   const omm_topk_mask& mask, int32_t* out, void* part) {
  TopkArgs a{};
  a.MG = static_cast<int>(MG);
  a.H = static_cast<int>(H);
  a.D = D;
  a.NC = static_cast<int>(NC);
  a.topk = topk;
  a.scale = scale;
  a.mk = to_dev(mask);
  a.out = out;
  a.part = static_cast<uint64_t*>(part);
  a.G = 1;
  return a;
}

void set_q(TopkArgs& a, const omm_view4& q) {
  a.q = q.data;
  a.qs0 = q.stride[0]; a.qs1 = q.stride[1]; a.qs2 = q.stride[2]; a.qs3 = q.stride[3];
}
void set_k(TopkArgs& a, const omm_view4& k) {
  a.k = k.data;
  a.ks0 = k.stride[0]; a.ks1 = k.stride[1]; a.ks2 = k.stride[2]; a.ks3 = k.stride[3];
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// topk > kMaxTopk: every row's scores go to the workspace ([B, MG, H, NC] fp32), then one
// workgroup per row selects (topk_large_kernel)
size_t large_ws_bytes(int64_t B, int64_t MG, int64_t H, int64_t NC) {
  return align256(static_cast<size_t>(B * MG * H) * static_cast<size_t>(NC) * sizeof(float));
}

int launch_large(const float* scores, int64_t B, int64_t MG, int64_t H, int64_t NC, int topk,
                 const omm_topk_mask& mask, int32_t* out, hipStream_t s) {
  const int64_t rows = B * MG * H;
  OMM_REQUIRE(rows <= 2147483647ll && MG <= 2147483647ll && NC <= 2147483647ll,
              OMM_EUNSUPPORTED, "top-k: %lld rows exceed the grid", (long long)rows);
  topk_large_kernel<<<static_cast<unsigned>(rows), kLargeThreads, 0, s>>>(
      scores, static_cast<int>(MG), static_cast<int>(H), static_cast<int>(NC), topk,
      to_dev(mask), out);
  return check_launch("top-k (topk > 128)");
}

// ---- MFMA path planning ---------------------------------------------------------------------
inline bool m2_view_ok(const omm_view4& v) {
  return v.stride[3] == 1 && v.stride[0] % 8 == 0 && v.stride[1] % 8 == 0 &&
         v.stride[2] % 8 == 0 && a16(v.data);
}
// 16-bit inputs, head dim 64 or 128, unit dim strides, 16-byte aligned rows, topk <= 16.
bool m2_ok(int32_t dtype, const omm_view4& q, const omm_view4& k, int topk) {
  if (dtype != OMM_BF16 && dtype != OMM_F16) return false;
  if (topk > 16) return false;
  const int64_t D = q.size[3];
  return (D == 64 || D == 128) && m2_view_ok(q) && m2_view_ok(k);
}

struct M2Plan {
  int span, nspan, rtiles;
  size_t ws_part;
};

// fused: one item per 16-row tile covers every column (q is pooled once).  Otherwise the columns
// are split into spans so that about 512 items (two per CU) run, and a merge kernel selects
// again over the spans' winners.
M2Plan m2_plan(int64_t B, int64_t MG, int64_t H, int64_t NC, int topk, bool fused) {
  M2Plan p{};
  p.rtiles = static_cast<int>(cdiv64(MG, kM2Rows));
  const int64_t tiles = B * H * p.rtiles;
  int64_t nspan = cdiv64(NC, kM2SpanCap);
  if (!fused && tiles * nspan < 512)
    nspan = std::max(nspan, std::min(cdiv64(512, tiles), cdiv64(NC, 256)));
  int64_t span = (cdiv64(NC, nspan) + 15) / 16 * 16;
  if (span < 16) span = 16;
  p.span = static_cast<int>(span);
  p.nspan = static_cast<int>(std::max<int64_t>(1, cdiv64(NC, span)));
  p.ws_part = p.nspan > 1 ? static_cast<size_t>(B * MG * H) * p.nspan * topk * sizeof(uint64_t) : 0;
  return p;
}

bool m2_fused_ok(int64_t B, int64_t MG, int64_t H, int64_t NC) {
  return NC <= kM2SpanCap && B * H * cdiv64(MG, kM2Rows) >= 256;
}

template <typename T, int D, bool FUSED>
int launch_m2_typed(M2Args a, int64_t B, int64_t H, const M2Plan& p, hipStream_t s) {
  const size_t lds = m2_lds_bytes(p.span, D);
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&topk_mfma_kernel<T, D, FUSED>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return set_error(OMM_EHIP, "top-k: LDS attribute: %s", hipGetErrorString(e));
  }
  a.span = p.span;
  a.nspan = p.nspan;
  a.rtiles = p.rtiles;
  a.o_qs = static_cast<uint32_t>(align16(static_cast<size_t>(kM2Rows) * m2_pitch(p.span) * 4));
  a.o_sv = static_cast<uint32_t>(align16(a.o_qs + static_cast<size_t>(kM2Rows) * (D + 8) * 2));
  a.o_tv = static_cast<uint32_t>(a.o_sv + static_cast<size_t>(kM2Waves) * kSurvCap * 8);
  const int64_t items = B * H * p.nspan * p.rtiles;
  OMM_REQUIRE(items <= 2147483647ll, OMM_EUNSUPPORTED, "top-k: grid too large");
  topk_mfma_kernel<T, D, FUSED><<<static_cast<unsigned>(items), kM2Threads, lds, s>>>(a);
  int rc = check_launch("top-k (mfma)");
  if (rc != OMM_OK || p.nspan == 1) return rc;
  const int64_t rows = B * a.MG * H;
  topk_merge_kernel<<<static_cast<unsigned>(cdiv64(rows, kWaves)), kThreads, 0, s>>>(
      a.part, a.out, rows, p.nspan, a.topk, a.NC);
  return check_launch("top-k merge");
}

template <bool FUSED>
int launch_m2(int32_t dtype, int D, M2Args a, int64_t B, int64_t H, const M2Plan& p,
              hipStream_t s) {
  if (dtype == OMM_BF16)
    return D == 128 ? launch_m2_typed<bf16_t, 128, FUSED>(a, B, H, p, s)
                    : launch_m2_typed<bf16_t, 64, FUSED>(a, B, H, p, s);
  return D == 128 ? launch_m2_typed<f16_t, 128, FUSED>(a, B, H, p, s)
                  : launch_m2_typed<f16_t, 64, FUSED>(a, B, H, p, s);
}

M2Args m2_args(const omm_view4& q, const omm_view4& k, int64_t MG, int64_t H, int64_t NC,
               int topk, float scale, const omm_topk_mask& mask, int32_t* out, void* part,
               float* dump) {
  M2Args a{};
  a.q = q.data; a.qs0 = q.stride[0]; a.qs1 = q.stride[1]; a.qs2 = q.stride[2];
  a.k = k.data; a.ks0 = k.stride[0]; a.ks1 = k.stride[1]; a.ks2 = k.stride[2];
  a.MG = static_cast<int>(MG);
  a.H = static_cast<int>(H);
  a.NC = static_cast<int>(NC);
  a.topk = topk;
  a.scale = scale;
  a.mk = to_dev(mask);
  a.out = out;
  a.part = static_cast<uint64_t*>(part);
  a.dump = dump;
  a.G = 1;
  return a;
}

}  // namespace
}  // namespace omm

extern "C" size_t omm_topk_workspace_bytes(int64_t B, int64_t MG, int64_t H, int64_t NC,
                                           int32_t topk) {
  if (B <= 0 || MG <= 0 || H <= 0 || NC <= 0 || topk < 1 || topk > omm::kLargeTopkCap) return 0;
  if (topk > omm::kMaxTopk) return omm::large_ws_bytes(B, MG, H, NC);
  // the split plan does not depend on the head dim beyond the LDS cap; use the smallest cap
  // (fp32, D = 256) so the answer covers every dtype and head dim
  size_t ws = 0;
  for (int esize : {2, 4})
    for (int D : {64, 128, 256})
      for (bool scores : {false, true})
        ws = std::max(ws, omm::make_plan(B, MG, H, NC, topk, D, esize, scores, false).ws_part);
  return std::max(ws, omm::m2_plan(B, MG, H, NC, topk, false).ws_part);
}

extern "C" int omm_topk(const omm_view4* q, const omm_view4* k, int32_t dtype, int32_t topk,
                        float scale, const omm_topk_mask* mask, int32_t* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE(q != nullptr && k != nullptr, OMM_EINVAL, "omm_topk: null argument");
  int rc = check_mask(mask);
  if (rc) return rc;
  const int64_t B = q->size[0], MG = q->size[1], H = q->size[2], D = q->size[3], NC = k->size[1];
  OMM_REQUIRE(k->size[0] == B && k->size[2] == H && k->size[3] == D, OMM_EINVAL,
              "omm_topk: incompatible q [%lld,%lld,%lld,%lld] and k [%lld,%lld,%lld,%lld]",
              (long long)B, (long long)MG, (long long)H, (long long)D, (long long)k->size[0],
              (long long)k->size[1], (long long)k->size[2], (long long)k->size[3]);
  OMM_REQUIRE(D >= 1 && D <= 256, OMM_EUNSUPPORTED, "omm_topk: head dim must be in [1, 256], got %lld",
              (long long)D);
  const int es = esize_of(dtype);
  rc = check_sizes(B, MG, H, NC, topk, static_cast<int>(D), es, false);
  if (rc) return rc;
  if (B == 0 || MG == 0 || H == 0) return OMM_OK;  // empty output: out may be null
  OMM_REQUIRE(out != nullptr, OMM_EINVAL, "omm_topk: null out");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (NC == 0) return fill_i32(out, B * MG * H * topk, -1, s);
  if (m2_ok(dtype, *q, *k, topk)) {
    const M2Plan p = m2_plan(B, MG, H, NC, topk, false);
    OMM_REQUIRE(p.ws_part <= workspace_bytes && (p.ws_part == 0 || workspace != nullptr),
                OMM_EWORKSPACE, "omm_topk: workspace of %zu bytes required, got %zu", p.ws_part,
                workspace_bytes);
    const M2Args a = m2_args(*q, *k, MG, H, NC, topk, scale, *mask, out, workspace, nullptr);
    return launch_m2<false>(dtype, static_cast<int>(D), a, B, H, p, s);
  }
  if (topk > kMaxTopk) {  // scores to the workspace, then the per-row selection
    const size_t need = large_ws_bytes(B, MG, H, NC);
    OMM_REQUIRE(workspace != nullptr && need <= workspace_bytes, OMM_EWORKSPACE,
                "omm_topk: workspace of %zu bytes required, got %zu", need, workspace_bytes);
    float* sc = static_cast<float*>(workspace);
    const Plan p = make_plan(B, MG, H, NC, topk, static_cast<int>(D), es, false, false);
    TopkArgs a = base_args(MG, H, NC, static_cast<int>(D), topk, scale, *mask, out, nullptr);
    set_q(a, *q);
    set_k(a, *k);
    a.vec = vec_ok(*q, es) && vec_ok(*k, es);
    a.dump = sc;
    rc = launch_typed<kModePooled>(dtype, a, B, MG, H, p, static_cast<int>(D), s);
    if (rc) return rc;
    return launch_large(sc, B, MG, H, NC, topk, *mask, out, s);
  }
  const Plan p = make_plan(B, MG, H, NC, topk, static_cast<int>(D), es, false, false);
  OMM_REQUIRE(p.ws_part <= workspace_bytes && (p.ws_part == 0 || workspace != nullptr),
              OMM_EWORKSPACE, "omm_topk: workspace of %zu bytes required, got %zu", p.ws_part,
              workspace_bytes);
  TopkArgs a = base_args(MG, H, NC, static_cast<int>(D), topk, scale, *mask, out, workspace);
  set_q(a, *q);
  set_k(a, *k);
  a.vec = vec_ok(*q, es) && vec_ok(*k, es);
  return launch_typed<kModePooled>(dtype, a, B, MG, H, p, static_cast<int>(D), s);
}

extern "C" size_t omm_topk_fused_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D,
                                                 int64_t NC, int32_t group_size, int32_t topk,
                                                 int32_t dtype) {
  using namespace omm;
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0 || NC <= 0 || group_size < 1 || topk < 1 ||
      topk > omm::kLargeTopkCap)
    return 0;
  const int64_t MG = cdiv64(T, group_size);
  const int es = esize_of(dtype);
  const size_t pooled = align256(static_cast<size_t>(B * MG * H * D) * es);
  return pooled + omm_topk_workspace_bytes(B, MG, H, NC, topk);
}

namespace omm {
namespace {
int topk_fused_impl(const omm_view4* q, const omm_view4* k, int32_t dtype, int32_t group_size,
                    int32_t topk, float scale, const omm_topk_mask* mask, int32_t* out,
                    float* dump, void* workspace, size_t workspace_bytes, void* stream) {
  OMM_REQUIRE(q != nullptr && k != nullptr, OMM_EINVAL, "omm_topk_fused: null argument");
  OMM_REQUIRE(group_size >= 1, OMM_EINVAL, "omm_topk_fused: group_size must be >= 1, got %d",
              group_size);
  int rc = check_mask(mask);
  if (rc) return rc;
  for (int i = 0; i < 4; ++i)
    OMM_REQUIRE(q->size[i] >= 0 && q->stride[i] >= 0 && k->stride[i] >= 0, OMM_EINVAL,
                "omm_topk_fused: negative size or stride");
  const int64_t B = q->size[0], T = q->size[1], H = q->size[2], D = q->size[3], NC = k->size[1];
  const int64_t MG = cdiv64(T, group_size);
  OMM_REQUIRE(k->size[0] == B && k->size[2] == H && k->size[3] == D, OMM_EINVAL,
              "omm_topk_fused: incompatible q [%lld,%lld,%lld,%lld] and k [%lld,%lld,%lld,%lld]",
              (long long)B, (long long)T, (long long)H, (long long)D, (long long)k->size[0],
              (long long)k->size[1], (long long)k->size[2], (long long)k->size[3]);
  OMM_REQUIRE(D >= 1 && D <= 256, OMM_EUNSUPPORTED,
              "omm_topk_fused: head dim must be in [1, 256], got %lld", (long long)D);
  OMM_REQUIRE(T <= 2147483647ll, OMM_EUNSUPPORTED, "omm_topk_fused: too many tokens");
  const int es = esize_of(dtype);
  rc = check_sizes(B, MG, H, NC, topk, static_cast<int>(D), es, false);
  if (rc) return rc;
  if (B == 0 || MG == 0 || H == 0) return OMM_OK;  // empty output: out may be null
  OMM_REQUIRE(out != nullptr, OMM_EINVAL, "omm_topk_fused: null out");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (NC == 0) return fill_i32(out, B * MG * H * topk, -1, s);
  OMM_REQUIRE(q->data != nullptr && k->data != nullptr, OMM_EINVAL, "omm_topk_fused: null data");

  if (m2_ok(dtype, *q, *k, topk)) {
    if (m2_fused_ok(B, MG, H, NC)) {
      const M2Plan p = m2_plan(B, MG, H, NC, topk, true);
      M2Args a = m2_args(*q, *k, MG, H, NC, topk, scale, *mask, out, nullptr, dump);
      a.T_len = static_cast<int>(T);
      a.G = group_size;
      return launch_m2<true>(dtype, static_cast<int>(D), a, B, H, p, s);
    }
    // few rows or a long key history: pool once into the workspace, then column spans
    const size_t pooled_bytes = align256(static_cast<size_t>(B * MG * H * D) * es);
    const M2Plan p = m2_plan(B, MG, H, NC, topk, false);
    const size_t need = pooled_bytes + p.ws_part;
    OMM_REQUIRE(workspace != nullptr && need <= workspace_bytes, OMM_EWORKSPACE,
                "omm_topk_fused: workspace of %zu bytes required, got %zu", need, workspace_bytes);
    omm_view4 pooled{};
    pooled.data = workspace;
    pooled.size[0] = B; pooled.size[1] = MG; pooled.size[2] = H; pooled.size[3] = D;
    pooled.stride[3] = 1; pooled.stride[2] = D; pooled.stride[1] = H * D;
    pooled.stride[0] = MG * H * D;
    OMM_REQUIRE(MG <= 65535 && B <= 65535, OMM_EUNSUPPORTED, "omm_topk_fused: grid limit");
    rc = pool_launch(*q, pooled, dtype, group_size, s);
    if (rc) return rc;
    const M2Args a = m2_args(pooled, *k, MG, H, NC, topk, scale, *mask, out,
                             static_cast<unsigned char*>(workspace) + pooled_bytes, dump);
    return launch_m2<false>(dtype, static_cast<int>(D), a, B, H, p, s);
  }
  OMM_REQUIRE(dump == nullptr, OMM_EUNSUPPORTED,
              "omm_topk_fused_debug: the score dump exists on the MFMA path only (bf16 / f16, "
              "head dim 64 or 128, unit dim strides, 16-byte aligned rows)");

  if (topk > kMaxTopk) {  // pool, scores to the workspace, then the per-row selection
    const size_t pooled_bytes = align256(static_cast<size_t>(B * MG * H * D) * es);
    const size_t need = pooled_bytes + large_ws_bytes(B, MG, H, NC);
    OMM_REQUIRE(workspace != nullptr && need <= workspace_bytes, OMM_EWORKSPACE,
                "omm_topk_fused: workspace of %zu bytes required, got %zu", need, workspace_bytes);
    omm_view4 pooled{};
    pooled.data = workspace;
    pooled.size[0] = B; pooled.size[1] = MG; pooled.size[2] = H; pooled.size[3] = D;
    pooled.stride[3] = 1; pooled.stride[2] = D; pooled.stride[1] = H * D;
    pooled.stride[0] = MG * H * D;
    OMM_REQUIRE(MG <= 65535 && B <= 65535, OMM_EUNSUPPORTED, "omm_topk_fused: grid limit");
    rc = pool_launch(*q, pooled, dtype, group_size, s);
    if (rc) return rc;
    float* sc = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + pooled_bytes);
    const Plan p = make_plan(B, MG, H, NC, topk, static_cast<int>(D), es, false, false);
    TopkArgs a = base_args(MG, H, NC, static_cast<int>(D), topk, scale, *mask, out, nullptr);
    set_q(a, pooled);
    set_k(a, *k);
    a.vec = vec_ok(pooled, es) && vec_ok(*k, es);
    a.dump = sc;
    rc = launch_typed<kModePooled>(dtype, a, B, MG, H, p, static_cast<int>(D), s);
    if (rc) return rc;
    return launch_large(sc, B, MG, H, NC, topk, *mask, out, s);
  }

  const bool vec = vec_ok(*q, es) && vec_ok(*k, es);
  if (vec && fused_ok(B, MG, H, NC, static_cast<int>(D), es)) {
    const Plan p = make_plan(B, MG, H, NC, topk, static_cast<int>(D), es, false, true);
    TopkArgs a = base_args(MG, H, NC, static_cast<int>(D), topk, scale, *mask, out, nullptr);
    set_q(a, *q);
    set_k(a, *k);
    a.vec = 1;
    a.T_len = static_cast<int>(T);
    a.G = group_size;
    return launch_typed<kModeFused>(dtype, a, B, MG, H, p, static_cast<int>(D), s);
  }
  // few rows or a long key history: pool once into the workspace, then the split kernel
  const size_t pooled_bytes = align256(static_cast<size_t>(B * MG * H * D) * es);
  const Plan p = make_plan(B, MG, H, NC, topk, static_cast<int>(D), es, false, false);
  const size_t need = pooled_bytes + p.ws_part;
  OMM_REQUIRE(workspace != nullptr && need <= workspace_bytes, OMM_EWORKSPACE,
              "omm_topk_fused: workspace of %zu bytes required, got %zu", need, workspace_bytes);
  omm_view4 pooled{};
  pooled.data = workspace;
  pooled.size[0] = B; pooled.size[1] = MG; pooled.size[2] = H; pooled.size[3] = D;
  pooled.stride[3] = 1; pooled.stride[2] = D; pooled.stride[1] = H * D; pooled.stride[0] = MG * H * D;
  OMM_REQUIRE(MG <= 65535 && B <= 65535, OMM_EUNSUPPORTED, "omm_topk_fused: grid limit");
  rc = pool_launch(*q, pooled, dtype, group_size, s);
  if (rc) return rc;
  TopkArgs a = base_args(MG, H, NC, static_cast<int>(D), topk, scale, *mask, out,
                         static_cast<unsigned char*>(workspace) + pooled_bytes);
  set_q(a, pooled);
  set_k(a, *k);
  a.vec = vec_ok(pooled, es) && vec_ok(*k, es);
  return launch_typed<kModePooled>(dtype, a, B, MG, H, p, static_cast<int>(D), s);
}
}  // namespace
}  // namespace omm

extern "C" int omm_topk_fused(const omm_view4* q, const omm_view4* k, int32_t dtype,
                              int32_t group_size, int32_t topk, float scale,
                              const omm_topk_mask* mask, int32_t* out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return omm::topk_fused_impl(q, k, dtype, group_size, topk, scale, mask, out, nullptr, workspace,
                              workspace_bytes, stream);
}

extern "C" int omm_topk_fused_debug(const omm_view4* q, const omm_view4* k, int32_t dtype,
                                    int32_t group_size, int32_t topk, float scale,
                                    const omm_topk_mask* mask, int32_t* out, float* scores,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE(scores != nullptr, OMM_EINVAL, "omm_topk_fused_debug: null scores");
  return topk_fused_impl(q, k, dtype, group_size, topk, scale, mask, out, scores, workspace,
                         workspace_bytes, stream);
}

extern "C" int omm_topk_from_scores(const float* scores, int64_t B, int64_t MG, int64_t H,
                                    int64_t NC, int32_t topk, const omm_topk_mask* mask,
                                    int32_t* out, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  using namespace omm;
  int rc = check_mask(mask);
  if (rc) return rc;
  rc = check_sizes(B, MG, H, NC, topk, 128, 4, true);
  if (rc) return rc;
  if (B == 0 || MG == 0 || H == 0) return OMM_OK;  // empty output: out may be null
  OMM_REQUIRE(out != nullptr, OMM_EINVAL, "omm_topk_from_scores: null output");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (NC == 0) return fill_i32(out, B * MG * H * topk, -1, s);
  OMM_REQUIRE(scores != nullptr, OMM_EINVAL, "omm_topk_from_scores: null scores");
  if (topk > kMaxTopk) return launch_large(scores, B, MG, H, NC, topk, *mask, out, s);
  const Plan p = make_plan(B, MG, H, NC, topk, 128, 4, true, false);
  OMM_REQUIRE(p.ws_part <= workspace_bytes && (p.ws_part == 0 || workspace != nullptr),
              OMM_EWORKSPACE, "omm_topk_from_scores: workspace of %zu bytes required, got %zu",
              p.ws_part, workspace_bytes);
  TopkArgs a = base_args(MG, H, NC, 128, topk, 0.0f, *mask, out, workspace);
  a.scores = scores;
  return launch_core<float, kModeScores>(a, B, MG, H, p, 128, s);
}

// ---- allocation-free variant of omm_topk_fused ----------------------------------------------
// For callers that cannot allocate device memory (code under HIP graph capture, serving loops
// that forbid hipMalloc): the workspace is a fixed array in the code object's device memory,
// one copy per GPU, held until the process ends.
namespace omm {
namespace {

constexpr size_t kTopkScratchBytes = size_t(8) << 20;

// In host code this name stands for the symbol, not a device address: host code reaches the
// array only through the per-device address hipGetSymbolAddress returns (scratch_of_stream).
static __device__ __align__(256) unsigned char scratch[kTopkScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices] = {};

// The scratch address on the device that owns `stream` (the current device for the null
// stream), looked up once per device with that device current.
int scratch_of_stream(hipStream_t stream, void** addr) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(OMM_EHIP, "omm_topk_fused_noalloc: device of the stream: %s",
                     hipGetErrorString(e));
  OMM_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, OMM_EUNSUPPORTED,
              "omm_topk_fused_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess || p == nullptr)
      return set_error(OMM_EHIP, "omm_topk_fused_noalloc: scratch address on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return OMM_OK;
}

}  // namespace
}  // namespace omm

extern "C" size_t omm_topk_fused_noalloc_max_bytes(void) { return omm::kTopkScratchBytes; }

extern "C" int omm_topk_fused_noalloc(const omm_view4* q, const omm_view4* k, int32_t dtype,
                                      int32_t group_size, int32_t topk, float scale,
                                      const omm_topk_mask* mask, int32_t* out, void* stream) {
  using namespace omm;
  OMM_REQUIRE(q != nullptr && k != nullptr, OMM_EINVAL, "omm_topk_fused_noalloc: null argument");
  const size_t need = omm_topk_fused_workspace_bytes(q->size[0], q->size[1], q->size[2],
                                                     q->size[3], k->size[1], group_size, topk,
                                                     dtype);
  OMM_REQUIRE(need <= kTopkScratchBytes, OMM_EWORKSPACE,
              "omm_topk_fused_noalloc: this call needs %zu bytes of scratch but the static "
              "scratch holds %zu; call omm_topk_fused with a workspace instead",
              need, kTopkScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_of_stream(static_cast<hipStream_t>(stream), &ws);
  if (rc != OMM_OK) return rc;
  return omm_topk_fused(q, k, dtype, group_size, topk, scale, mask, out, ws, kTopkScratchBytes,
                        stream);
}
