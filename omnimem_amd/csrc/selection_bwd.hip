// Selection attention backward over dense K / V: delta, dQ, the block -> query-group index, and
// dK / dV.
//
// Reference semantics: cuda_backend/csrc/selection_bwd.cu:18-163 (dQ: delta = rowsum(out * dO)
// in fp32, P recomputed as exp(s * scale - lse), dS = P (dP - delta) scale, dQ = dS K),
// :164-306 (dK / dV: one owner per key block walks the query groups that selected it, no
// atomics), inverted_index.cu:13-34 (which (group, slot) pairs a block receives: id in range,
// block not after the group's chunk when causal), bwd_common.cuh:33-60 (partial tail blocks,
// per-token chunk-causal prefix), :1329-1407 (dK / dV of never-selected tokens are 0, results
// in the K / V dtype).
//
// gfx950 design (bf16 / f16), three launches:
//   sel_bwd_dq_kernel    one workgroup = 64 queries of one group, 2 waves x 32 queries, the same
//                        block walk and LDS-DMA K / V tiles as the forward kernel.  Per key tile:
//                        S^T = K Q^T and dP^T = V dO^T (K and V rows from LDS, Q^T and dO^T held
//                        in registers), P = 2^(s c2 - lse log2 e), dS = P (dP - delta) scale,
//                        then dQ^T += K^T dS^T with dS^T straight from the accumulator layout and
//                        K^T from ds_read_b64_tr_b16.  Writes dQ and delta.
//   sel_bwd_index_kernel one workgroup per (b, h, 64 blocks): counts, scans and scatters every
//                        valid (group, slot) pair into per-block buckets (CSR), in (group, slot) order,
//                        so the dK / dV sums have a fixed order (the reference's buckets are in
//                        atomic arrival order).
//   sel_bwd_dkv_kernel   one workgroup per (b, h, block, 64-key tile), 2 waves x 32 keys.  K and V
//                        of its keys stay in registers as MFMA operands; the queries of each
//                        bucket group stream through LDS (64-row Q / dO tiles by LDS DMA, double
//                        buffered, with their lse and delta).  S = Q K^T, dP = dO V^T, then
//                        dV += P^T dO and dK += dS^T Q with P^T / dS^T from the accumulator
//                        layout and dO / Q from transposed LDS reads.  Every token of every block
//                        is written (0 when no group selected it).
#include <type_traits>

#include "sel_common.h"

namespace omm {
namespace {

// 8 packed 16-bit values of two rows -> fp32 dot product (fixed order, fp32 products).
template <typename QT> __device__ __forceinline__ float dot8(uint4 a, uint4 b);
template <> __device__ __forceinline__ float dot8<bf16_t>(uint4 a, uint4 b) {
  const uint32_t x[4] = {a.x, a.y, a.z, a.w}, y[4] = {b.x, b.y, b.z, b.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += __builtin_bit_cast(float, x[i] << 16) * __builtin_bit_cast(float, y[i] << 16);
    s += __builtin_bit_cast(float, x[i] & 0xffff0000u) * __builtin_bit_cast(float, y[i] & 0xffff0000u);
  }
  return s;
}
template <> __device__ __forceinline__ float dot8<f16_t>(uint4 a, uint4 b) {
  const uint32_t x[4] = {a.x, a.y, a.z, a.w}, y[4] = {b.x, b.y, b.z, b.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const _Float16 x0 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(x[i]));
    const _Float16 x1 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(x[i] >> 16));
    const _Float16 y0 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(y[i]));
    const _Float16 y1 = __builtin_bit_cast(_Float16, static_cast<uint16_t>(y[i] >> 16));
    s += static_cast<float>(x0) * static_cast<float>(y0);
    s += static_cast<float>(x1) * static_cast<float>(y1);
  }
  return s;
}

// -lse in the log2 domain; -inf for a row with no visible token (its P is then 0).
__device__ __forceinline__ float neg_lse2(float l) { return l == kNegInf ? kNegInf : -l * kLog2e; }

// ---- dQ -------------------------------------------------------------------------------------
constexpr int kDqThreads = 128;

template <typename QT, typename Acc, int D>
__global__ __launch_bounds__(kDqThreads, 2) void sel_bwd_dq_kernel(
    View4<const QT> q, View4<const QT> o, View4<const QT> dout, View4<QT> dq,
    const float* __restrict__ lse, float* __restrict__ delta, float* __restrict__ nl2out, Acc acc,
    int M, int H, int G, int MG, int T, int chunk, float scale, int nsub) {
  using DG = DmaGeom<D>;
  constexpr int ROWB = DG::ROWB, CPR = DG::CPR, TK = DG::TK, RPI = DG::RPI;
  constexpr int NT = DG::NT, NU = DG::NU, SD = DG::SD, ND = DG::ND;
  __shared__ __align__(16) char lds[4][8192];  // K buffers 0, 1; V buffers 2, 3

  const int tid = static_cast<int>(threadIdx.x), lane = lane_id(), w = tid / kWave;
  const int l16 = lane & 15, j4 = lane >> 4;
  const int total = static_cast<int>(gridDim.x);
  int wi = xcd_remap(static_cast<int>(blockIdx.x), total);
  const int sub = wi % nsub; wi /= nsub;
  const int g = wi % MG; wi /= MG;
  const int h = wi % H;
  const int b = wi / H;

  const int m0 = g * G + sub * 64;
  const int m_end = min(min(g * G + G, M), m0 + 64);
  const int qc = (g * G) / chunk;

  // Q^T and dO^T operands of this wave's 2 query blocks (row m0 + 32 w + 16 x + l16, dims
  // 32 s + 8 j4 ..), each query's delta (a 4-lane-group reduction) and -lse log2 e
  bool q_ok[2];
  uint4 qb[2][SD], db[2][SD];
  float nl2[2], dl[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int mq = m0 + 32 * w + 16 * x + l16;
    q_ok[x] = mq < m_end;
    float part = 0.0f;
#pragma unroll
    for (int s = 0; s < SD; ++s) {
      if (q_ok[x]) {
        qb[x][s] = *reinterpret_cast<const uint4*>(q.at(b, mq, h, 32 * s + 8 * j4));
        db[x][s] = *reinterpret_cast<const uint4*>(dout.at(b, mq, h, 32 * s + 8 * j4));
        part += dot8<QT>(*reinterpret_cast<const uint4*>(o.at(b, mq, h, 32 * s + 8 * j4)),
                         db[x][s]);
      } else {
        qb[x][s] = make_uint4(0, 0, 0, 0);
        db[x][s] = make_uint4(0, 0, 0, 0);
      }
    }
    part += __shfl_xor(part, 16, kWave);
    part += __shfl_xor(part, 32, kWave);
    dl[x] = part;
    const int64_t li = (static_cast<int64_t>(b) * H + h) * M + mq;
    nl2[x] = q_ok[x] ? neg_lse2(lse[li]) : kNegInf;
    if (q_ok[x] && j4 == 0) {
      delta[li] = part;
      nl2out[li] = nl2[x];
    }
  }
  const float c2 = scale * kLog2e;
  // dO^T negated (sign bits, exact) and delta as the accumulator input: the dP^T MFMAs then
  // give delta - dP directly, and dS = -P (delta - dP) costs one multiply per score
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int s = 0; s < SD; ++s) {
      db[x][s].x ^= 0x80008000u;
      db[x][s].y ^= 0x80008000u;
      db[x][s].z ^= 0x80008000u;
      db[x][s].w ^= 0x80008000u;
    }
  const f32x4 dlv[2] = {f32x4{dl[0], dl[0], dl[0], dl[0]}, f32x4{dl[1], dl[1], dl[1], dl[1]}};

  // LDS read offsets inside a tile buffer; K and V rows are swizzled by swz_v (K is read both as
  // rows and transposed; measured on gfx950 swz_v serves both read kinds best).  K / V row
  // operand (t, s): row 16 t + l16, chunk 4 s + j4.  K^T operand (u, half, i): row 32 u +
  // 16 half + 4 j4 + (l16 >> 2), dims 16 i + 4 (l16 & 3) .. +3 (ds_read_b64_tr_b16 hands lane
  // l16 dim 16 i + l16 of 4 keys).
  int koff[SD], ktoff[ND];
#pragma unroll
  for (int s = 0; s < SD; ++s) koff[s] = l16 * ROWB + (((4 * s + j4) ^ DG::swz_v(l16)) << 4);
  {
    const int kr = 4 * j4 + (l16 >> 2), km = l16 & 3;
#pragma unroll
    for (int i = 0; i < ND; ++i)
      ktoff[i] = kr * ROWB + (((2 * i + (km >> 1)) ^ DG::swz_v(kr)) << 4) + ((km & 1) << 3);
  }

  f32x4 acc_dq[2][ND];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int i = 0; i < ND; ++i) acc_dq[x][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  WaveWalk<Acc, TK> wk;
  wk.start(acc, b, g, h, T, qc);
  int n_cur = 0;
  int kdo[4], vdo[4];
  int rsk = 0, rsv = 0;
  if (wk.valid) {
    rsk = static_cast<int>(wk.br.sk) * 2;
    rsv = static_cast<int>(wk.br.sv) * 2;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int row = (4 * w + jj) * RPI + lane / CPR, c = lane % CPR;
      kdo[jj] = row * rsk + ((c ^ DG::swz_v(row)) << 4);
      vdo[jj] = row * rsv + ((c ^ DG::swz_v(row)) << 4);
    }
    copy_part<Acc>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(wk.tok0) * rsk, rsk, wk.n,
             lds[0], w, kdo);
    copy_part<Acc>(static_cast<const char*>(wk.br.v) + static_cast<int64_t>(wk.tok0) * rsv, rsv, wk.n,
             lds[2], w, vdo);
    n_cur = wk.n;
    wk.advance(acc, b, g, h, T, qc);
  }
  __builtin_amdgcn_s_waitcnt(0);

  // one key tile in LDS buffers BI, a compile-time constant so that LDS addresses are a lane
  // offset plus an immediate
  auto step = [&](auto BIc) -> bool {
    constexpr int BI = decltype(BIc)::value;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int n_nx = 0;
    if (wk.valid) {
      copy_part<Acc>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(wk.tok0) * rsk, rsk,
               wk.n, lds[BI ^ 1], w, kdo);
      copy_part<Acc>(static_cast<const char*>(wk.br.v) + static_cast<int64_t>(wk.tok0) * rsv, rsv,
               wk.n, lds[2 + (BI ^ 1)], w, vdo);
      n_nx = wk.n;
      wk.advance(acc, b, g, h, T, qc);
    }
    const char* Kt = lds[BI];
    const char* Vt = lds[2 + BI];

    // S^T = K Q^T and dP^T = V dO^T: lane holds keys 16 t + 4 j4 + r of query l16
    f32x4 s4[2][NT], p4[2][NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      s4[0][t] = s4[1][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      p4[0][t] = dlv[0];
      p4[1][t] = dlv[1];
#pragma unroll
      for (int s = 0; s < SD; ++s) {
        const uint4 a = *reinterpret_cast<const uint4*>(Kt + koff[s] + 16 * t * ROWB);
        s4[0][t] = Mfma<QT>::run(a, qb[0][s], s4[0][t]);
        s4[1][t] = Mfma<QT>::run(a, qb[1][s], s4[1][t]);
        const uint4 av = *reinterpret_cast<const uint4*>(Vt + koff[s] + 16 * t * ROWB);
        p4[0][t] = Mfma<QT>::run(av, db[0][s], p4[0][t]);
        p4[1][t] = Mfma<QT>::run(av, db[1][s], p4[1][t]);
      }
    }
    // dS / scale = P (dP - delta), P = 2^e, e = s c2 - lse log2 e (the scale multiplies the dQ
    // sums once at the end).  Keys past n_cur are not visible: a wave-uniform branch taken by
    // partial tiles only sets their e to -inf, so P = 0 whatever the sign of c2 (a negative
    // scale makes c2 negative: -inf in s would give e = +inf).
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) s4[x][t][r] = __builtin_fmaf(s4[x][t][r], c2, nl2[x]);
    if (n_cur < TK) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (16 * t + 4 * j4 + r >= n_cur) s4[0][t][r] = s4[1][t][r] = kNegInf;
    }
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          s4[x][t][r] = -(__builtin_amdgcn_exp2f(s4[x][t][r]) * p4[x][t][r]);
    // dQ^T += K^T dS^T; k-slot e of lane group j4 is key 32 u + 4 j4 + e (e < 4) or
    // 32 u + 16 + 4 j4 + (e - 4), for both operands
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      uint4 sb[2];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        sb[x] = make_uint4(Mfma<QT>::pack2(s4[x][2 * u][0], s4[x][2 * u][1]),
                           Mfma<QT>::pack2(s4[x][2 * u][2], s4[x][2 * u][3]),
                           Mfma<QT>::pack2(s4[x][2 * u + 1][0], s4[x][2 * u + 1][1]),
                           Mfma<QT>::pack2(s4[x][2 * u + 1][2], s4[x][2 * u + 1][3]));
#pragma unroll
      for (int i = 0; i < ND; ++i) {
        const uint2 lo = lds_read_tr16(Kt + ktoff[i] + (32 * u) * ROWB);
        const uint2 hi = lds_read_tr16(Kt + ktoff[i] + (32 * u + 16) * ROWB);
        const uint4 ka = make_uint4(lo.x, lo.y, hi.x, hi.y);
        acc_dq[0][i] = Mfma<QT>::run(ka, sb[0], acc_dq[0][i]);
        acc_dq[1][i] = Mfma<QT>::run(ka, sb[1], acc_dq[1][i]);
      }
    }
    n_cur = n_nx;
    return n_cur > 0;
  };
  if (n_cur > 0)
    while (step(std::integral_constant<int, 0>{}) && step(std::integral_constant<int, 1>{})) {
    }

  // lane holds dQ[query l16][dims 16 i + 4 j4 + r]
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    if (!q_ok[x]) continue;
    const int mq = m0 + 32 * w + 16 * x + l16;
    QT* op = dq.at(b, mq, h, 0);
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      uint2 w2;
      w2.x = Mfma<QT>::pack2(acc_dq[x][i][0] * scale, acc_dq[x][i][1] * scale);
      w2.y = Mfma<QT>::pack2(acc_dq[x][i][2] * scale, acc_dq[x][i][3] * scale);
      *reinterpret_cast<uint2*>(op + 16 * i + 4 * j4) = w2;
    }
  }
}

// ---- block -> query-group index --------------------------------------------------------------
constexpr int kIdxThreads = 512;
constexpr int kIdxWaves = kIdxThreads / kWave;
constexpr int kIdxBuckets = 64;  // buckets per workgroup

// Bucket of (group g, slot t) of row (b, h), or -1 when the pair reaches no key.  Ids at or past
// the row's limit (NS, or n_blocks[h] when that is smaller) reach none.
struct PairBucket {
  const int32_t* ids;
  int64_t is0, is1, is2, is3;
  int T, NS, bs, chunk, G;
  bool causal;
  const int32_t* n_blocks;  // per-head bound, or nullptr
  __device__ __forceinline__ int32_t id(int b, int h, int p) const {
    const int g = p / T, t = p - g * T;
    return ids[b * is0 + g * is1 + h * is2 + t * is3];
  }
  __device__ __forceinline__ int limit(int h) const {
    return n_blocks != nullptr ? min(NS, n_blocks[h]) : NS;
  }
  __device__ __forceinline__ int bucket(int32_t bid, int p, int lim) const {
    const int g = p / T;
    if (bid < 0 || bid >= lim) return -1;
    // 32-bit unsigned: bid * bs < N + bs and g * G < M + G, with M, N < 2^31
    if (causal && (static_cast<uint32_t>(bid) * static_cast<uint32_t>(bs)) / static_cast<uint32_t>(chunk) >
                      (static_cast<uint32_t>(g) * static_cast<uint32_t>(G)) / static_cast<uint32_t>(chunk))
      return -1;
    return bid;
  }
};

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// offsets: [B*H][NS+1]; groups: [B*H][MG*T] (bucket j of row r is groups[r][offsets[r][j] ..
// offsets[r][j+1]), ascending (group, slot)).  One workgroup per (row, 64 buckets lo .. lo+63):
// wave w of 8 takes the w-th eighth of the row's pairs in order.  Pass 1 counts, per wave, the pairs
// of each of the workgroup's buckets and those below lo; the scan then gives every bucket its
// offset and every (wave, bucket) its first place.  Pass 2 walks each wave's pairs 64 at a time;
// a pair's place is its (wave, bucket) cursor plus the number of lower lanes of the batch in the
// same bucket, read from a 64-bit per-(wave, bucket) mask.  Waves touch only their own counters
// and masks, so the passes need no workgroup barrier inside.
__global__ __launch_bounds__(kIdxThreads) void sel_bwd_index_kernel(
    PairBucket pb, int H, int P, int nrange, int32_t* __restrict__ offsets,
    int32_t* __restrict__ groups) {
  constexpr int NW = kIdxWaves, R = kIdxBuckets;
  static_assert(R == kWave, "one bucket per lane in the scan");
  __shared__ int cur[NW][R];                   // counts, then cursors
  __shared__ unsigned long long msk[NW][R];
  __shared__ int below[NW];
  const int row = static_cast<int>(blockIdx.x) / nrange;
  const int rg = static_cast<int>(blockIdx.x) - row * nrange;
  const int b = row / H, h = row - (row / H) * H;
  const int tid = static_cast<int>(threadIdx.x), lane = lane_id(), w = tid / kWave;
  const int NS = pb.NS, lo = rg * R, nb = min(R, NS - lo);
  int32_t* off = offsets + static_cast<int64_t>(row) * (NS + 1);
  int32_t* grp = groups + static_cast<int64_t>(row) * P;
  const int per = (P + NW - 1) / NW;
  const int p0 = min(P, w * per), p1 = min(P, p0 + per);
  const int lim = pb.limit(h);

  // a wave's pairs are read PL per lane at a time, all loads in flight together
  constexpr int PL = 16;
  auto load = [&](int c0, int (&kk)[PL]) {
    int32_t raw[PL];
#pragma unroll
    for (int j = 0; j < PL; ++j) raw[j] = pb.id(b, h, min(c0 + j * kWave + lane, p1 - 1));
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int p = c0 + j * kWave + lane;
      kk[j] = p < p1 ? pb.bucket(raw[j], p, lim) : -1;
    }
  };

  cur[w][lane] = 0;
  msk[w][lane] = 0ull;
  wave_sync_lds();
  int nbelow = 0;
  for (int c0 = p0; c0 < p1; c0 += PL * kWave) {
    int kk[PL];
    load(c0, kk);
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int k = kk[j];
      if (k >= 0 && k < lo) ++nbelow;
      else if (k >= lo && k < lo + nb) atomicAdd(&cur[w][k - lo], 1);
    }
  }
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) nbelow += __shfl_xor(nbelow, d, kWave);
  if (lane == 0) below[w] = nbelow;
  __syncthreads();

  if (w == 0) {  // lane = bucket lo + lane
    int c[NW], tot = 0, base = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      c[j] = cur[j][lane];
      tot += c[j];
      base += below[j];
    }
    int incl = tot;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int y = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += y;
    }
    int run = base + incl - tot;
    if (lane < nb) off[lo + lane] = run;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      cur[j][lane] = run;
      run += c[j];
    }
    if (lo + R >= NS && lane == kWave - 1) off[NS] = base + incl;
  }
  __syncthreads();

  for (int c0 = p0; c0 < p1; c0 += PL * kWave) {
    int kk[PL];
    load(c0, kk);
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      if (c0 + j * kWave >= p1) break;  // wave-uniform
      const int p = c0 + j * kWave + lane;
      const int k = kk[j] >= 0 ? kk[j] - lo : -1;
      const bool in = k >= 0 && k < nb;
      if (in) atomicOr(&msk[w][k], 1ull << lane);
      wave_sync_lds();
      unsigned long long m = 0ull;
      int r = 0;
      if (in) {
        m = msk[w][k];
        r = __builtin_popcountll(m & ((1ull << lane) - 1ull));
        grp[cur[w][k] + r] = p / pb.T;
      }
      wave_sync_lds();
      if (in && r == 0) {
        cur[w][k] += __builtin_popcountll(m);
        msk[w][k] = 0ull;
      }
      wave_sync_lds();
    }
  }
}

// ---- dK / dV ----------------------------------------------------------------------------------
// Workgroup = 4 waves over one 64-key tile: wave w owns keys 16 w .. 16 w + 15 (one MFMA column
// block) for every query of every item.  Its K / V operands and fp32 dK / dV sums take ~100
// registers, so two waves share each SIMD (the workgroup's 66 KiB of LDS allows two workgroups
// per CU) and one wave's LDS and memory waits are covered by the other's work.  The item's lse arrives
// already as -lse log2 e (written by the dQ kernel), and the softmax scale of dK is applied once
// to the sums.
constexpr int kKvThreads = 256;

// One dword per lane: lane L's float at base + 4 L (lanes at or past nvalid read 0) into LDS
// dst + 4 L, issued like dma_part (inline asm, ordered by the kernel's own waits).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_f32x64(const float* base, int nvalid, float* dst) {
  const i32x4 r = buffer_desc(base, 4 * nvalid);
  const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
      static_cast<int>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)))));
  const int off = 4 * lane_id();
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(off), "s"(r)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// ---- dK / dV targets --------------------------------------------------------------------------
// One key tile (up to 64 tokens) of one (b, h, block): element pointers of its first K / V row and
// first dK / dV row, element strides, its row count and the token id of its first row (used by the
// chunk-causal mask only).
template <typename KT, typename GT>
struct KvTile {
  const KT* k;
  const KT* v;
  GT* dk;
  GT* dv;
  int64_t k_sn, k_sd, v_sn, v_sd, dk_sn, dk_sd, dv_sn, dv_sd;
  int nk, t0;
};

// Dense K / V and dK / dV [B, N, H, D]: block bid is tokens bid*bs .. min(bid*bs + bs, N).
template <typename QT>
struct DenseGrad {
  using KT = QT;
  using GT = QT;
  static constexpr bool kMayMisalign = false;  // 16-byte rows checked on the host
  View4<const QT> k, v;
  View4<QT> dk, dv;
  int N, bs;
  __device__ __forceinline__ bool tile(int b, int h, int bid, int kt, KvTile<QT, QT>& r) const {
    const int t0 = bid * bs + 64 * kt;
    const int nk = min(min(bs - 64 * kt, 64), N - t0);
    if (nk <= 0) return false;
    r = KvTile<QT, QT>{k.at(b, t0, h), v.at(b, t0, h), dk.at(b, t0, h), dv.at(b, t0, h),
                       k.s1, k.s3, v.s1, v.s3, dk.s1, dk.s3, dv.s1, dv.s3, nk, t0};
    return true;
  }
};

// Raw block addresses of a pointer-table caller (bf16 K / V, fp32 dK / dV scratch), from [H, MAXB]
// base tables: with blocks_per_chunk > 0 the base of (h, bid / blocks_per_chunk) plus
// (bid % blocks_per_chunk) in-chunk block strides, else the base of (h, bid); plus b batch
// strides.  A block is skipped (nothing read or written) when bid is at or past n_blocks[h] (if
// given) or past the table, or when any of its four bases is 0 (reference contract:
// bwd_common.cuh:66-121).  Every block holds bs tokens.
struct PtrGrad {
  using KT = bf16_t;
  using GT = float;
  static constexpr bool kMayMisalign = true;  // any 2-byte aligned K / V address is accepted
  const int64_t* base_k;
  const int64_t* base_v;
  const int64_t* base_dk;
  const int64_t* base_dv;
  int64_t bsh, bsc;  // element strides of the base tables
  int64_t max_base;
  const int32_t* n_blocks;
  int64_t batch_kv, batch_dkv, chunk_kv, chunk_dkv;  // bytes
  int64_t s_bn, s_bd, s_dbn, s_dbd;                  // element strides
  int bpc, bs;
  __device__ __forceinline__ bool tile(int b, int h, int bid, int kt, KvTile<bf16_t, float>& r) const {
    if (n_blocks != nullptr && bid >= n_blocks[h]) return false;
    const int64_t idx = bpc > 0 ? bid / bpc : bid;
    const int64_t loc = bpc > 0 ? bid - idx * bpc : 0;
    if (idx >= max_base) return false;
    const int64_t o = h * bsh + idx * bsc;
    const int64_t bk = base_k[o], bv = base_v[o], bdk = base_dk[o], bdv = base_dv[o];
    if (bk == 0 || bv == 0 || bdk == 0 || bdv == 0) return false;
    const int nk = min(bs - 64 * kt, 64);
    if (nk <= 0) return false;
    const int64_t okv = b * batch_kv + loc * chunk_kv, od = b * batch_dkv + loc * chunk_dkv;
    const int64_t row0 = 64 * static_cast<int64_t>(kt);
    r.k = reinterpret_cast<const bf16_t*>(static_cast<uintptr_t>(bk + okv)) + row0 * s_bn;
    r.v = reinterpret_cast<const bf16_t*>(static_cast<uintptr_t>(bv + okv)) + row0 * s_bn;
    r.dk = reinterpret_cast<float*>(static_cast<uintptr_t>(bdk + od)) + row0 * s_dbn;
    r.dv = reinterpret_cast<float*>(static_cast<uintptr_t>(bdv + od)) + row0 * s_dbn;
    r.k_sn = r.v_sn = s_bn;
    r.k_sd = r.v_sd = s_bd;
    r.dk_sn = r.dv_sn = s_dbn;
    r.dk_sd = r.dv_sd = s_dbd;
    r.nk = nk;
    r.t0 = 0;
    return true;
  }
};

// 8 consecutive 16-bit elements (unit stride) as one MFMA operand; a target that admits 2-byte
// aligned rows reads a misaligned row with 2-byte loads.
template <bool MIS>
__device__ __forceinline__ uint4 load_row8(const void* p) {
  if constexpr (MIS) {
    if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0u) {
      const uint16_t* e = static_cast<const uint16_t*>(p);
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = static_cast<uint32_t>(e[2 * i]) | (static_cast<uint32_t>(e[2 * i + 1]) << 16);
      return make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  return *static_cast<const uint4*>(p);
}

// 8 fp32 results of one row, dims d .. d + 7: 16-bit rows (unit stride, 16-byte aligned) get one
// packed 16-byte store; fp32 rows two 16-byte stores when contiguous and aligned, else 8 stores.
template <typename QT>
__device__ __forceinline__ void store_row8(QT* p, int64_t, const float4& x0, const float4& x1) {
  *reinterpret_cast<uint4*>(p) =
      make_uint4(Mfma<QT>::pack2(x0.x, x0.y), Mfma<QT>::pack2(x0.z, x0.w),
                 Mfma<QT>::pack2(x1.x, x1.y), Mfma<QT>::pack2(x1.z, x1.w));
}
__device__ __forceinline__ void store_row8(float* p, int64_t sd, const float4& x0,
                                           const float4& x1) {
  if (sd == 1 && (reinterpret_cast<uintptr_t>(p) & 15u) == 0u) {
    reinterpret_cast<float4*>(p)[0] = x0;
    reinterpret_cast<float4*>(p)[1] = x1;
    return;
  }
  const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i * sd] = x[i];
}

template <typename QT, int D, typename KG>
__global__ __launch_bounds__(kKvThreads, 2) void sel_bwd_dkv_kernel(
    View4<const QT> q, View4<const QT> dout, KG kg, const float* __restrict__ nl2,
    const float* __restrict__ delta, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ groups, int M, int H, int G, int MG, int T, int NS, int nkt,
    int chunk, bool causal, float scale, int nsub) {
  using DG = DmaGeom<D>;
  constexpr int ROWB = DG::ROWB, CPR = DG::CPR, RPI = DG::RPI;
  constexpr int SD = DG::SD, ND = DG::ND;
  constexpr int QB = 64 * ROWB;           // bytes of one 64-row Q or dO tile
  constexpr int NPC = QB / 4096;          // 4 KiB copy pieces per tile (4 copy instructions)
  constexpr int PPW = 2 * NPC / 4;        // pieces per wave (Q and dO pieces of both tiles)
  // [Q buffer 0, Q buffer 1, dO buffer 0, dO buffer 1][QB] then [buffer][lse, delta][64]
  __shared__ __align__(16) char smem[4 * QB + 2 * 2 * 64 * 4];

  const int tid = static_cast<int>(threadIdx.x), lane = lane_id(), w = tid / kWave;
  const int l16 = lane & 15, j4 = lane >> 4;
  // Work order.  A key block's work is the number of query groups that selected it; under a
  // causal chunk mask the early blocks are picked by many more groups than the late ones.  Units
  // u = (b, h, key tile) are split into P classes of blocks (bid mod P), P the smallest with U P a
  // multiple of 8, so that each XCD (workgroup id mod 8 under round-robin dispatch) gets U P / 8
  // whole classes of equal expected work.  An XCD runs its classes one after another, each with
  // its blocks ascending (heavy first), so the workgroups it holds at once share one head's
  // Q/dO tiles in its L2.  Blocks past the last full round of P come last, units fastest.
  const int id = static_cast<int>(blockIdx.x), U = static_cast<int>(gridDim.x) / NS;
  const int P = 8 / ((U & 7) == 0 ? 8 : (U & 3) == 0 ? 4 : (U & 1) == 0 ? 2 : 1);
  const int nb = NS / P, S = U * P / 8, treg = U * nb * P;
  int u, bid;
  if (id < treg) {
    const int x = id & 7, kk = id >> 3, su = x * S + kk / nb, bi = kk - (kk / nb) * nb;
    u = su / P;
    bid = bi * P + (su - u * P);
  } else {
    const int r = id - treg;
    u = r % U;
    bid = nb * P + r / U;
  }
  const int kt = u % nkt; u /= nkt;
  const int h = u % H;
  const int b = u / H;

  KvTile<typename KG::KT, typename KG::GT> tl;
  if (!kg.tile(b, h, bid, kt, tl)) return;
  const int t0 = tl.t0, nk = tl.nk;  // first token and tokens of the tile

  // K^T and V^T operands of this wave's key 16 w + l16, dims 32 s + 8 j4 ..
  uint4 kb[SD], vb[SD];
  {
    const int key = 16 * w + l16;
    const bool ok = key < nk;
#pragma unroll
    for (int s = 0; s < SD; ++s) {
      kb[s] = ok ? load_row8<KG::kMayMisalign>(tl.k + key * tl.k_sn + 32 * s + 8 * j4)
                 : make_uint4(0, 0, 0, 0);
      vb[s] = ok ? load_row8<KG::kMayMisalign>(tl.v + key * tl.v_sn + 32 * s + 8 * j4)
                 : make_uint4(0, 0, 0, 0);
    }
  }
  const float c2 = scale * kLog2e;

  // LDS offsets (Q and dO tiles share one layout, rows swizzled by swz_v, which depends on the
  // row modulo 8 only; measured on gfx950 it serves the b128 row reads as well as swz_k and the
  // transposed reads best).  Row operand (hq, x, s): row 32 hq + 16 x + l16, 16-byte chunk
  // (4 s + j4) ^ swz_v(l16) = rx ^ 4 s.  Transposed operand (hq, half, i): row 32 hq +
  // 16 half + tr, tr = 4 j4 + (l16 >> 2), chunk (2 i + (tm >> 1)) ^ swz_v(tr) =
  // 2 (i ^ tx) + (tm >> 1) (swz_v is even), plus 8 bytes for odd tm = l16 & 3.  Offsets are
  // formed at each use from these few registers.
  const int rbase = l16 * ROWB;
  const int rx = j4 ^ DG::swz_v(l16);
  const int tr = 4 * j4 + (l16 >> 2), tm = l16 & 3;
  const int tbase = tr * ROWB + ((tm >> 1) << 4) + ((tm & 1) << 3);
  const int tx = DG::swz_v(tr) >> 1;
  auto roff = [&](int s) { return rbase + ((rx ^ (4 * s)) << 4); };
  auto troff = [&](int i) { return tbase + ((i ^ tx) << 5); };
  // copy pieces of this wave: piece p = w + 4 pp of [Q pieces 0 .. NPC-1, dO pieces 0 .. NPC-1];
  // instruction jj of piece pc copies rows (4 pc + jj) RPI + lane / CPR, whose row modulo 8
  // (and so swizzle) does not depend on pc
  const int rsq = static_cast<int>(q.s1) * 2, rsd = static_cast<int>(dout.s1) * 2;
  const int crow = lane / CPR;
  int csw[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) csw[jj] = ((lane % CPR) ^ DG::swz_v(jj * RPI + crow)) << 4;

  // dK / scale and dV of keys 16 w + 4 j4 + r, dims 16 i + l16
  f32x4 acc_dk[ND], acc_dv[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) acc_dk[i] = acc_dv[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t orow = (static_cast<int64_t>(b) * H + h) * (NS + 1);
  const int e0 = offsets[orow + bid], e1 = offsets[orow + bid + 1];
  const int32_t* grp = groups + (static_cast<int64_t>(b) * H + h) * (static_cast<int64_t>(MG) * T);
  const int nitems = (e1 - e0) * nsub;
  const int64_t lrow = (static_cast<int64_t>(b) * H + h) * M;

  // item i = (bucket entry i / nsub, 64-query part i % nsub): its first query, queries and
  // visible keys of this tile; find() returns the next item with work at or after i
  struct Item {
    int i, q0, nq, nv;
  };
  // bucket entries held in a VGPR, 64 at a time (lane j: entry gwin + j), read with readlane
  int gwin = -64, gv = 0;
  auto group_of = [&](int e) -> int {
    if ((e & ~63) != gwin) {
      gwin = e & ~63;
      gv = gwin + lane < e1 - e0 ? grp[e0 + gwin + lane] : 0;
    }
    return __builtin_amdgcn_readlane(gv, e & 63);
  };
  auto find = [&](int i) -> Item {
    for (; i < nitems; ++i) {
      const int e = i / nsub, part = i - (i / nsub) * nsub;
      const int g = group_of(e);
      const int q0 = g * G + 64 * part;
      const int nq = min(min(g * G + G, M) - q0, 64);
      int nv = nk;
      if (causal) {
        const int64_t lim = static_cast<int64_t>((g * G) / chunk + 1) * chunk - t0;
        nv = lim < nv ? static_cast<int>(lim > 0 ? lim : 0) : nv;
      }
      if (nq > 0 && nv > 0) return Item{i, q0, nq, nv};
    }
    return Item{nitems, 0, 0, 0};
  };
  auto issue = [&](const Item& it, int buf) {
    const char* qbase = reinterpret_cast<const char*>(q.at(b, it.q0, h, 0));
    const char* dbase = reinterpret_cast<const char*>(dout.at(b, it.q0, h, 0));
#pragma unroll
    for (int pp = 0; pp < PPW; ++pp) {
      const int piece = w + 4 * pp, pc = piece % NPC;
      const bool isq = piece < NPC;
      const int rs = isq ? rsq : rsd;
      int off[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) off[jj] = ((4 * pc + jj) * RPI + crow) * rs + csw[jj];
      dma_part(isq ? qbase : dbase, rs, it.nq, smem + (isq ? buf : 2 + buf) * QB, pc, off);
    }
    if (w < 2)
      dma_f32x64((w == 0 ? nl2 : delta) + lrow + it.q0, it.nq,
                 reinterpret_cast<float*>(smem + 4 * QB) + (buf * 2 + w) * 64);
  };

  Item cur = find(0);
  if (cur.i < nitems) issue(cur, 0);
  __builtin_amdgcn_s_waitcnt(0);

  int BI = 0;
  while (cur.i < nitems) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const Item nx = find(cur.i + 1);
    if (nx.i < nitems) issue(nx, BI ^ 1);
    const char* Qt = smem + BI * QB;
    const char* Dt = smem + (2 + BI) * QB;
    const float* Ls = reinterpret_cast<const float*>(smem + 4 * QB) + BI * 128;
    const float* Ds = Ls + 64;
    const bool kv = 16 * w + l16 < cur.nv;

#pragma unroll
    for (int hq = 0; hq < 2; ++hq) {  // queries 32 hq .. 32 hq + 31
      // S = Q K^T and dP = dO V^T: lane holds queries 32 hq + 16 x + 4 j4 + r of key 16 w + l16
      f32x4 s4[2], p4[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        s4[x] = p4[x] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < SD; ++s) {
          const int ro = roff(s) + (32 * hq + 16 * x) * ROWB;
          s4[x] = Mfma<QT>::run(*reinterpret_cast<const uint4*>(Qt + ro), kb[s], s4[x]);
          p4[x] = Mfma<QT>::run(*reinterpret_cast<const uint4*>(Dt + ro), vb[s], p4[x]);
        }
      }
      // P and dS / scale; padded query rows have zero Q / dO and lse = delta = 0, so they add
      // nothing
      float pv[2][4], dsv[2][4];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const float4 L4 = *reinterpret_cast<const float4*>(Ls + 32 * hq + 16 * x + 4 * j4);
        const float4 D4 = *reinterpret_cast<const float4*>(Ds + 32 * hq + 16 * x + 4 * j4);
        const float Lr[4] = {L4.x, L4.y, L4.z, L4.w}, Dr[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s4[x][r], c2, Lr[r]));
          p = kv ? p : 0.0f;
          pv[x][r] = p;
          dsv[x][r] = p * (p4[x][r] - Dr[r]);
        }
      }
      // k-slot e of lane group j4 is query 32 hq + 4 j4 + e (e < 4) or 32 hq + 16 + 4 j4 +
      // (e - 4): x = 0 rows then x = 1 rows
      const uint4 pa = make_uint4(Mfma<QT>::pack2(pv[0][0], pv[0][1]),
                                  Mfma<QT>::pack2(pv[0][2], pv[0][3]),
                                  Mfma<QT>::pack2(pv[1][0], pv[1][1]),
                                  Mfma<QT>::pack2(pv[1][2], pv[1][3]));
      const uint4 sa = make_uint4(Mfma<QT>::pack2(dsv[0][0], dsv[0][1]),
                                  Mfma<QT>::pack2(dsv[0][2], dsv[0][3]),
                                  Mfma<QT>::pack2(dsv[1][0], dsv[1][1]),
                                  Mfma<QT>::pack2(dsv[1][2], dsv[1][3]));
      // dV += P^T dO and dK += dS^T Q: B operands dO / Q rows 32 hq + 4 j4 + y (+16), dim
      // 16 i + l16, from transposed reads
#pragma unroll
      for (int i = 0; i < ND; ++i) {
        const int to = troff(i) + 32 * hq * ROWB;
        const uint2 dlo = lds_read_tr16(Dt + to), dhi = lds_read_tr16(Dt + to + 16 * ROWB);
        const uint2 qlo = lds_read_tr16(Qt + to), qhi = lds_read_tr16(Qt + to + 16 * ROWB);
        acc_dv[i] = Mfma<QT>::run(pa, make_uint4(dlo.x, dlo.y, dhi.x, dhi.y), acc_dv[i]);
        acc_dk[i] = Mfma<QT>::run(sa, make_uint4(qlo.x, qlo.y, qhi.x, qhi.y), acc_dk[i]);
      }
    }
    cur = nx;
    BI ^= 1;
  }

  // stage the fp32 key rows ([dK, dV][64 keys][D], 64 KiB: the Q / dO buffers) so that the
  // whole workgroup converts 8 values at a time (packed conversions) and stores 16 bytes per
  // lane; no copy is in flight here (the last item issued none)
  float* stage = reinterpret_cast<float*>(smem);
  static_assert(4 * QB >= 2 * 64 * D * 4, "staging area");
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int key = 16 * w + 4 * j4 + r;
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      stage[key * D + 16 * i + l16] = acc_dk[i][r] * scale;
      stage[(64 + key) * D + 16 * i + l16] = acc_dv[i][r];
    }
  }
  __syncthreads();
  constexpr int CH = D / 8;  // 8-element chunks per row
  for (int c = tid; c < 2 * 64 * CH; c += kKvThreads) {
    const int row = c / CH, ch = c - (c / CH) * CH;
    const int key = row & 63;
    if (key >= nk) continue;
    const float4 x0 = *reinterpret_cast<const float4*>(stage + row * D + 8 * ch);
    const float4 x1 = *reinterpret_cast<const float4*>(stage + row * D + 8 * ch + 4);
    if (row < 64)
      store_row8(tl.dk + key * tl.dk_sn + 8 * ch * tl.dk_sd, tl.dk_sd, x0, x1);
    else
      store_row8(tl.dv + key * tl.dv_sn + 8 * ch * tl.dv_sd, tl.dv_sd, x0, x1);
  }
}

// ---- VALU kernels (fp32 arithmetic; any element type, head dim <= 256 and strides) ------------
// The reference's FP32 SIMT kernels (selection_bwd.cu:18-306) in the same roles: dQ walks a
// group's blocks with 4 lanes per query (DQ dims each, dot products reduced over the 4 lanes),
// dK / dV owns a 64-key tile with 4 lanes per key and walks the bucket groups' queries through
// LDS.  P = exp(s scale - lse) in the natural-log domain, as the reference computes it.
constexpr int kVKeys = 32;   // keys per LDS tile (dQ)
constexpr int kVQ = 16;      // queries per LDS tile (dK / dV)

template <typename QT, typename Acc, int DQ>
__global__ __launch_bounds__(256) void sel_bwd_dq_valu_kernel(
    View4<const QT> q, View4<const QT> o, View4<const QT> dout, View4<QT> dq,
    const float* __restrict__ lse, float* __restrict__ delta, float* __restrict__ nl2out, Acc acc,
    int M, int H, int D, int G, int MG, int T, int chunk, float scale, int nsub, int64_t kv_sd) {
  constexpr int DP = 4 * DQ;
  __shared__ float Ks[kVKeys * DP];
  __shared__ float Vs[kVKeys * DP];
  using KVT = typename Acc::KV;
  const int tid = threadIdx.x;
  const int total = static_cast<int>(gridDim.x);
  int wi = xcd_remap(static_cast<int>(blockIdx.x), total);
  const int sub = wi % nsub; wi /= nsub;
  const int g = wi % MG; wi /= MG;
  const int h = wi % H;
  const int b = wi / H;
  const int m0 = g * G + sub * 64;
  const int m_end = min(min(g * G + G, M), m0 + 64);
  const int qc = (g * G) / chunk;
  const int qi = tid >> 2, part = tid & 3;
  const int my_q = m0 + qi;
  const bool q_ok = my_q < m_end;
  const int d0 = part * DQ;

  float qr[DQ], dr[DQ], acc_q[DQ];
  float dl = 0.0f;
#pragma unroll
  for (int i = 0; i < DQ; ++i) {
    const int d = d0 + i;
    const bool ok = q_ok && d < D;
    qr[i] = ok ? to_f32<QT>(*q.at(b, my_q, h, d)) : 0.0f;
    dr[i] = ok ? to_f32<QT>(*dout.at(b, my_q, h, d)) : 0.0f;
    dl += ok ? to_f32<QT>(*o.at(b, my_q, h, d)) * dr[i] : 0.0f;
    acc_q[i] = 0.0f;
  }
  dl += __shfl_xor(dl, 1, kWave);
  dl += __shfl_xor(dl, 2, kWave);
  const int64_t li = (static_cast<int64_t>(b) * H + h) * M + my_q;
  const float L = q_ok ? lse[li] : kNegInf;
  if (q_ok && part == 0) {
    delta[li] = dl;
    nl2out[li] = neg_lse2(L);
  }
  for (TileIt it = first_tile(acc, b, g, h, T, qc, 0); it.valid;) {
    for (int k0 = 0; k0 < it.n; k0 += kVKeys) {
      const int nk = min(kVKeys, it.n - k0);
      __syncthreads();
      for (int i = tid; i < kVKeys * DP; i += 256) {
        const int kk = i / DP, d = i - kk * DP;
        float kvv = 0.0f, vvv = 0.0f;
        if (kk < nk && d < D) {
          const int64_t row = it.tok0 + k0 + kk;
          kvv = kv_elem<KVT>(it.br.k, row * it.br.sk + d * kv_sd, it.br.scale_k);
          vvv = kv_elem<KVT>(it.br.v, row * it.br.sv + d * kv_sd, it.br.scale_v);
        }
        Ks[i] = kvv;
        Vs[i] = vvv;
      }
      __syncthreads();
      for (int kk = 0; kk < nk; ++kk) {
        float s = 0.0f, dp = 0.0f;
#pragma unroll
        for (int i = 0; i < DQ; ++i) {
          s = __builtin_fmaf(qr[i], Ks[kk * DP + d0 + i], s);
          dp = __builtin_fmaf(dr[i], Vs[kk * DP + d0 + i], dp);
        }
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        dp += __shfl_xor(dp, 1, kWave);
        dp += __shfl_xor(dp, 2, kWave);
        const float p = L == kNegInf ? 0.0f : expf(s * scale - L);
        const float ds = p * (dp - dl) * scale;
#pragma unroll
        for (int i = 0; i < DQ; ++i) acc_q[i] = __builtin_fmaf(ds, Ks[kk * DP + d0 + i], acc_q[i]);
      }
    }
    it = next_tile(acc, it, b, g, h, T, qc);
  }
  if (q_ok) {
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      const int d = d0 + i;
      if (d < D) *dq.at(b, my_q, h, d) = from_f32<QT>(acc_q[i]);
    }
  }
}

template <typename QT, int DQ, typename KG>
__global__ __launch_bounds__(256) void sel_bwd_dkv_valu_kernel(
    View4<const QT> q, View4<const QT> dout, KG kg, const float* __restrict__ lse,
    const float* __restrict__ delta, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ groups, int M, int H, int D, int G, int MG, int T, int NS,
    int nkt, int chunk, bool causal, float scale) {
  constexpr int DP = 4 * DQ;
  __shared__ float Qs[kVQ * DP];
  __shared__ float Ds[kVQ * DP];
  __shared__ float Ls[kVQ], Dl[kVQ];
  const int tid = threadIdx.x;
  // Work order.  A key block's work is the number of query groups that selected it; under a
  // causal chunk mask the early blocks are picked by many more groups than the late ones.  Units
  // u = (b, h, key tile) are split into P classes of blocks (bid mod P), P the smallest with U P a
  // multiple of 8, so that each XCD (workgroup id mod 8 under round-robin dispatch) gets U P / 8
  // whole classes of equal expected work.  An XCD runs its classes one after another, each with
  // its blocks ascending (heavy first), so the workgroups it holds at once share one head's
  // Q/dO tiles in its L2.  Blocks past the last full round of P come last, units fastest.
  const int id = static_cast<int>(blockIdx.x), U = static_cast<int>(gridDim.x) / NS;
  const int P = 8 / ((U & 7) == 0 ? 8 : (U & 3) == 0 ? 4 : (U & 1) == 0 ? 2 : 1);
  const int nb = NS / P, S = U * P / 8, treg = U * nb * P;
  int u, bid;
  if (id < treg) {
    const int x = id & 7, kk = id >> 3, su = x * S + kk / nb, bi = kk - (kk / nb) * nb;
    u = su / P;
    bid = bi * P + (su - u * P);
  } else {
    const int r = id - treg;
    u = r % U;
    bid = nb * P + r / U;
  }
  const int kt = u % nkt; u /= nkt;
  const int h = u % H;
  const int b = u / H;
  using KT = typename KG::KT;
  using GT = typename KG::GT;
  KvTile<KT, GT> tl;
  if (!kg.tile(b, h, bid, kt, tl)) return;
  const int t0 = tl.t0, nk = tl.nk;
  const int key = tid >> 2, part = tid & 3, d0 = part * DQ;
  const bool k_ok = key < nk;

  float kr[DQ], vr[DQ], acc_k[DQ], acc_v[DQ];
#pragma unroll
  for (int i = 0; i < DQ; ++i) {
    const int d = d0 + i;
    const bool ok = k_ok && d < D;
    kr[i] = ok ? to_f32<KT>(tl.k[key * tl.k_sn + d * tl.k_sd]) : 0.0f;
    vr[i] = ok ? to_f32<KT>(tl.v[key * tl.v_sn + d * tl.v_sd]) : 0.0f;
    acc_k[i] = acc_v[i] = 0.0f;
  }
  const int64_t orow = (static_cast<int64_t>(b) * H + h) * (NS + 1);
  const int e0 = offsets[orow + bid], e1 = offsets[orow + bid + 1];
  const int32_t* grp = groups + (static_cast<int64_t>(b) * H + h) * (static_cast<int64_t>(MG) * T);
  const int64_t lrow = (static_cast<int64_t>(b) * H + h) * M;
  for (int e = e0; e < e1; ++e) {
    const int g = grp[e];
    const int q_begin = g * G, q_end = min(g * G + G, M);
    int nv = nk;
    if (causal) {
      const int64_t lim = static_cast<int64_t>((g * G) / chunk + 1) * chunk - t0;
      nv = lim < nv ? static_cast<int>(lim > 0 ? lim : 0) : nv;
    }
    if (nv <= 0) continue;  // workgroup-uniform
    const bool kv = key < nv;
    for (int q0 = q_begin; q0 < q_end; q0 += kVQ) {
      const int nq = min(kVQ, q_end - q0);
      __syncthreads();
      for (int i = tid; i < kVQ * DP; i += 256) {
        const int qq = i / DP, d = i - qq * DP;
        const bool ok = qq < nq && d < D;
        Qs[i] = ok ? to_f32<QT>(*q.at(b, q0 + qq, h, d)) : 0.0f;
        Ds[i] = ok ? to_f32<QT>(*dout.at(b, q0 + qq, h, d)) : 0.0f;
      }
      if (tid < kVQ) {
        Ls[tid] = tid < nq ? lse[lrow + q0 + tid] : kNegInf;
        Dl[tid] = tid < nq ? delta[lrow + q0 + tid] : 0.0f;
      }
      __syncthreads();
      for (int qq = 0; qq < nq; ++qq) {
        float s = 0.0f, dp = 0.0f;
#pragma unroll
        for (int i = 0; i < DQ; ++i) {
          s = __builtin_fmaf(Qs[qq * DP + d0 + i], kr[i], s);
          dp = __builtin_fmaf(Ds[qq * DP + d0 + i], vr[i], dp);
        }
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        dp += __shfl_xor(dp, 1, kWave);
        dp += __shfl_xor(dp, 2, kWave);
        const float L = Ls[qq];
        const float p = (kv && L != kNegInf) ? expf(s * scale - L) : 0.0f;
        const float ds = p * (dp - Dl[qq]) * scale;
#pragma unroll
        for (int i = 0; i < DQ; ++i) {
          acc_k[i] = __builtin_fmaf(ds, Qs[qq * DP + d0 + i], acc_k[i]);
          acc_v[i] = __builtin_fmaf(p, Ds[qq * DP + d0 + i], acc_v[i]);
        }
      }
    }
  }
  if (k_ok) {
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      const int d = d0 + i;
      if (d < D) {
        tl.dk[key * tl.dk_sn + d * tl.dk_sd] = from_f32<GT>(acc_k[i]);
        tl.dv[key * tl.dv_sn + d * tl.dv_sd] = from_f32<GT>(acc_v[i]);
      }
    }
  }
}

// ---- host side ----------------------------------------------------------------------------------
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct BwdWs {
  size_t delta, nl2, offsets, groups, total;
};
// [delta (dense entry only) | -lse log2 e | CSR offsets | bucket lists (when dK / dV are computed)]
inline BwdWs bwd_ws(int64_t B, int64_t M, int64_t H, int64_t MG, int64_t T, int64_t NS,
                    bool with_delta = true, bool with_index = true) {
  BwdWs w;
  w.delta = 0;
  w.nl2 = with_delta ? align256(static_cast<size_t>(B * H * M) * 4) : 0;
  w.offsets = w.nl2 + align256(static_cast<size_t>(B * H * M) * 4);
  w.groups = w.offsets + (with_index ? align256(static_cast<size_t>(B * H * (NS + 1)) * 4) : 0);
  w.total = w.groups + (with_index ? align256(static_cast<size_t>(B * H * MG * T) * 4) : 0);
  return w;
}

inline bool aligned16b(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 16-byte rows with unit dim stride, element strides in multiples of 8, rows of at least D
// elements and 64 rows within the 32-bit tile offsets of the LDS copies.
inline bool rows16(const omm_view4& x, int64_t D) {
  return x.stride[3] == 1 && aligned16b(x.data) && x.stride[0] % 8 == 0 && x.stride[1] % 8 == 0 &&
         x.stride[2] % 8 == 0 && x.stride[1] >= D && 2 * x.stride[1] * 64 < (int64_t{1} << 31);
}

struct BwdArgs {
  const omm_view4 *q, *k, *v, *ids, *out, *dout, *dq, *dk, *dv;
  const float* lse;
  int bs, chunk, G;
  bool causal;
  float scale;
};

// Launches: dQ (and delta, -lse log2 e), the block -> group index, dK / dV.  MFMA kernels when
// D is 64 or 128 with 16-bit rows (DM = D), else the VALU kernels with DQ dims per lane.
template <typename QT, int DM, int DQ>
int sel_bwd_launch(const BwdArgs& a, char* ws, const BwdWs& L, hipStream_t s) {
  const omm_view4 &q = *a.q, &k = *a.k, &v = *a.v, &ids = *a.ids;
  const int B = static_cast<int>(q.size[0]), M = static_cast<int>(q.size[1]);
  const int H = static_cast<int>(q.size[2]), D = static_cast<int>(q.size[3]);
  const int N = static_cast<int>(k.size[1]);
  const int MG = static_cast<int>(ids.size[1]), T = static_cast<int>(ids.size[3]);
  const int bs = a.bs, G = a.G;
  const int NS = static_cast<int>(cdiv64(N, bs));
  const int nsub = (G + 63) / 64;
  const bool causal = a.causal;
  const int ch = causal ? a.chunk : 1;
  float* delta = reinterpret_cast<float*>(ws + L.delta);
  float* nl2 = reinterpret_cast<float*>(ws + L.nl2);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* groups = reinterpret_cast<int32_t*>(ws + L.groups);

  OMM_REQUIRE(ids_offsets_fit32(ids), OMM_EUNSUPPORTED,
              "omm_sel_bwd: block_indices must span fewer than 2^31 elements");
  OMM_REQUIRE(kv_offsets_fit32(k, v), OMM_EUNSUPPORTED,
              "omm_sel_bwd: a (batch, head) slice of k / v must span fewer than 2^32 elements");
  DenseAcc<QT> acc{make_view<const QT>(k), make_view<const QT>(v),
                   static_cast<const int32_t*>(ids.data), ids.stride[0], ids.stride[1],
                   ids.stride[2], ids.stride[3], N, bs, ch, causal};
  const int64_t dq_items = static_cast<int64_t>(B) * H * MG * nsub;
  const int nkt = (bs + 63) / 64;
  const int64_t kv_items = static_cast<int64_t>(B) * H * NS * nkt;
  OMM_REQUIRE(dq_items <= 2147483647ll && kv_items <= 2147483647ll, OMM_EUNSUPPORTED,
              "omm_sel_bwd: grid too large");
  if constexpr (DM > 0) {
    sel_bwd_dq_kernel<QT, DenseAcc<QT>, DM><<<static_cast<unsigned>(dq_items), kDqThreads, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.out), make_view<const QT>(*a.dout),
        make_view<QT>(*a.dq), a.lse, delta, nl2, acc, M, H, G, MG, T, ch, a.scale, nsub);
  } else {
    sel_bwd_dq_valu_kernel<QT, DenseAcc<QT>, DQ><<<static_cast<unsigned>(dq_items), 256, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.out), make_view<const QT>(*a.dout),
        make_view<QT>(*a.dq), a.lse, delta, nl2, acc, M, H, D, G, MG, T, ch, a.scale, nsub,
        k.stride[3]);
  }
  int rc = check_launch("selection backward (dq)");
  if (rc) return rc;

  PairBucket pb{static_cast<const int32_t*>(ids.data), ids.stride[0], ids.stride[1],
                ids.stride[2], ids.stride[3], T, NS, bs, ch, G, causal, nullptr};
  const int nrange = std::max(1, (NS + kIdxBuckets - 1) / kIdxBuckets);  // NS = 0: offsets[0] = 0
  sel_bwd_index_kernel<<<static_cast<unsigned>(B * H * nrange), kIdxThreads, 0, s>>>(
      pb, H, MG * T, nrange, offsets, groups);
  rc = check_launch("selection backward (index)");
  if (rc) return rc;

  if (kv_items == 0) return OMM_OK;
  const DenseGrad<QT> kg{make_view<const QT>(k), make_view<const QT>(v), make_view<QT>(*a.dk),
                         make_view<QT>(*a.dv), N, bs};
  if constexpr (DM > 0) {
    sel_bwd_dkv_kernel<QT, DM, DenseGrad<QT>><<<static_cast<unsigned>(kv_items), kKvThreads, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.dout), kg, nl2, delta, offsets, groups, M,
        H, G, MG, T, NS, nkt, ch, causal, a.scale, nsub);
  } else {
    sel_bwd_dkv_valu_kernel<QT, DQ, DenseGrad<QT>><<<static_cast<unsigned>(kv_items), 256, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.dout), kg, a.lse, delta, offsets, groups,
        M, H, D, G, MG, T, NS, nkt, ch, causal, a.scale);
  }
  return check_launch("selection backward (dk/dv)");
}

// Pointer-table backward: dQ over the forward's address tables (no chunk mask), then, when dK / dV
// are asked for, the block -> query-group index over ids bounded per head and dK / dV into the
// callers' fp32 scratch blocks.  MFMA kernels when DM > 0, else the VALU kernels with DQ dims per
// lane.  The MFMA dK / dV kernel's item order assumes nothing about which blocks are popular.
struct PtrBwdArgs {
  const omm_view4 *q, *out, *dout, *ids, *dq;
  const float* lse;
  float* delta;
  PtrAcc acc;
  PtrGrad kg;
  int bs, G, NS;
  bool dkv;
  float scale;
};

template <int DM, int DQ>
int sel_bwd_ptr_launch(const PtrBwdArgs& a, char* ws, const BwdWs& L, hipStream_t s) {
  using QT = bf16_t;
  const omm_view4 &q = *a.q, &ids = *a.ids;
  const int B = static_cast<int>(q.size[0]), M = static_cast<int>(q.size[1]);
  const int H = static_cast<int>(q.size[2]), D = static_cast<int>(q.size[3]);
  const int MG = static_cast<int>(ids.size[1]), T = static_cast<int>(ids.size[3]);
  const int G = a.G, NS = a.NS, nsub = (G + 63) / 64;
  float* nl2 = reinterpret_cast<float*>(ws + L.nl2);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
  int32_t* groups = reinterpret_cast<int32_t*>(ws + L.groups);
  const int64_t dq_items = static_cast<int64_t>(B) * H * MG * nsub;
  const int nkt = (a.bs + 63) / 64;
  const int64_t kv_items = static_cast<int64_t>(B) * H * NS * nkt;
  OMM_REQUIRE(dq_items <= 2147483647ll && kv_items <= 2147483647ll, OMM_EUNSUPPORTED,
              "omm_sel_bwd_ptr: grid too large");
  if constexpr (DM > 0) {
    sel_bwd_dq_kernel<QT, PtrAcc, DM><<<static_cast<unsigned>(dq_items), kDqThreads, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.out), make_view<const QT>(*a.dout),
        make_view<QT>(*a.dq), a.lse, a.delta, nl2, a.acc, M, H, G, MG, T, 1, a.scale, nsub);
  } else {
    sel_bwd_dq_valu_kernel<QT, PtrAcc, DQ><<<static_cast<unsigned>(dq_items), 256, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.out), make_view<const QT>(*a.dout),
        make_view<QT>(*a.dq), a.lse, a.delta, nl2, a.acc, M, H, D, G, MG, T, 1, a.scale, nsub,
        a.kg.s_bd);
  }
  int rc = check_launch("pointer selection backward (dq)");
  if (rc || !a.dkv || kv_items == 0) return rc;

  PairBucket pb{static_cast<const int32_t*>(ids.data), ids.stride[0], ids.stride[1],
                ids.stride[2], ids.stride[3], T, NS, a.bs, 1, G, false, a.kg.n_blocks};
  const int nrange = (NS + kIdxBuckets - 1) / kIdxBuckets;
  sel_bwd_index_kernel<<<static_cast<unsigned>(B * H * nrange), kIdxThreads, 0, s>>>(
      pb, H, MG * T, nrange, offsets, groups);
  rc = check_launch("pointer selection backward (index)");
  if (rc) return rc;
  if constexpr (DM > 0) {
    sel_bwd_dkv_kernel<QT, DM, PtrGrad><<<static_cast<unsigned>(kv_items), kKvThreads, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.dout), a.kg, nl2, a.delta, offsets, groups,
        M, H, G, MG, T, NS, nkt, 1, false, a.scale, nsub);
  } else {
    sel_bwd_dkv_valu_kernel<QT, DQ, PtrGrad><<<static_cast<unsigned>(kv_items), 256, 0, s>>>(
        make_view<const QT>(q), make_view<const QT>(*a.dout), a.kg, a.lse, a.delta, offsets,
        groups, M, H, D, G, MG, T, NS, nkt, 1, false, a.scale);
  }
  return check_launch("pointer selection backward (dk/dv)");
}

template <typename QT>
int sel_bwd_typed(const BwdArgs& a, bool mfma, char* ws, const BwdWs& L, hipStream_t s) {
  const int64_t D = a.q->size[3];
  if constexpr (sizeof(QT) == 2) {
    if (mfma && D == 128) return sel_bwd_launch<QT, 128, 0>(a, ws, L, s);
    if (mfma && D == 64) return sel_bwd_launch<QT, 64, 0>(a, ws, L, s);
  }
  if (D <= 64) return sel_bwd_launch<QT, 0, 16>(a, ws, L, s);
  if (D <= 128) return sel_bwd_launch<QT, 0, 32>(a, ws, L, s);
  return sel_bwd_launch<QT, 0, 64>(a, ws, L, s);
}

}  // namespace
}  // namespace omm

extern "C" size_t omm_sel_bwd_workspace_bytes(int64_t B, int64_t M, int64_t H, int64_t N,
                                              int32_t block_size, int32_t group_size, int64_t T) {
  if (B <= 0 || M <= 0 || H <= 0 || N < 0 || block_size < 1 || group_size < 1 || T < 1) return 0;
  const int64_t MG = omm::cdiv64(M, group_size), NS = omm::cdiv64(N, block_size);
  return omm::bwd_ws(B, M, H, MG, T, NS).total;
}

extern "C" int omm_sel_bwd(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                           const omm_view4* ids, const omm_view4* out, const float* lse,
                           const omm_view4* dout, int32_t dtype, int32_t block_size,
                           int32_t chunk_size, int32_t causal, int32_t group_size, float scale,
                           const omm_view4* dq, const omm_view4* dk, const omm_view4* dv,
                           void* workspace, size_t workspace_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE(q && k && v && ids && out && lse && dout && dq && dk && dv, OMM_EINVAL,
              "omm_sel_bwd: null argument");
  const int64_t B = q->size[0], M = q->size[1], H = q->size[2], D = q->size[3];
  const int64_t N = k->size[1];
  for (int i = 0; i < 4; ++i) {
    OMM_REQUIRE(out->size[i] == q->size[i] && dout->size[i] == q->size[i] &&
                    dq->size[i] == q->size[i],
                OMM_EINVAL, "omm_sel_bwd: out, d_out and dq must have q's shape");
    OMM_REQUIRE(v->size[i] == k->size[i] && dk->size[i] == k->size[i] && dv->size[i] == k->size[i],
                OMM_EINVAL, "omm_sel_bwd: v, dk and dv must have k's shape");
  }
  OMM_REQUIRE(k->size[0] == B && k->size[2] == H && k->size[3] == D, OMM_EINVAL,
              "omm_sel_bwd: expected k/v [B,N,H,D] compatible with q");
  OMM_REQUIRE(group_size >= 1 && block_size >= 1 && chunk_size >= 1, OMM_EINVAL,
              "omm_sel_bwd: group_size, block_size and chunk_size must be >= 1");
  const int64_t MG = cdiv64(M, group_size);
  OMM_REQUIRE(ids->size[0] == B && ids->size[1] == MG && ids->size[2] == H && ids->size[3] >= 1,
              OMM_EINVAL, "omm_sel_bwd: block_indices must be [%lld,%lld,%lld,T>=1]", (long long)B,
              (long long)MG, (long long)H);
  OMM_REQUIRE(N <= 2147483647ll && M <= 2147483647ll && MG * ids->size[3] <= 2147483647ll &&
                  B * H * MG * ids->size[3] <= 2147483647ll,
              OMM_EUNSUPPORTED, "omm_sel_bwd: sizes exceed the int32 index range");
  if (B == 0 || M == 0 || H == 0) return OMM_OK;
  const int64_t T = ids->size[3];
  const BwdWs L = bwd_ws(B, M, H, MG, T, cdiv64(N, block_size));
  OMM_REQUIRE(workspace != nullptr && workspace_bytes >= L.total &&
                  (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
              OMM_EWORKSPACE, "omm_sel_bwd: workspace of %zu bytes (256-byte aligned) required",
              L.total);
  OMM_REQUIRE(D >= 1 && D <= 256, OMM_EUNSUPPORTED, "omm_sel_bwd: head dim must be in [1, 256] "
              "(got %lld)", (long long)D);
  OMM_REQUIRE(__builtin_isfinite(scale), OMM_EINVAL, "omm_sel_bwd: scale must be finite");
  // MFMA kernels: 16-bit rows of head dim 64 / 128, 16-byte aligned, and a non-zero scale;
  // everything else runs the VALU kernels (k and v then need one dim stride)
  bool rows_ok = true;
  for (const omm_view4* x : {q, k, v, out, dout, dq, dk, dv}) rows_ok = rows_ok && rows16(*x, D);
  const bool mfma = (dtype == OMM_BF16 || dtype == OMM_F16) && (D == 64 || D == 128) && rows_ok &&
                    scale != 0.0f;
  OMM_REQUIRE(mfma || k->stride[3] == v->stride[3], OMM_EUNSUPPORTED,
              "omm_sel_bwd: k and v need the same dim stride");
  char* ws = static_cast<char*>(workspace);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const BwdArgs a{q, k, v, ids, out, dout, dq, dk, dv, lse, block_size, chunk_size, group_size,
                  causal != 0, scale};
  switch (dtype) {
    case OMM_BF16: return sel_bwd_typed<bf16_t>(a, mfma, ws, L, s);
    case OMM_F16: return sel_bwd_typed<f16_t>(a, mfma, ws, L, s);
    case OMM_F32: return sel_bwd_typed<float>(a, false, ws, L, s);
    default: return set_error(OMM_EINVAL, "omm_sel_bwd: unsupported dtype %d", dtype);
  }
}

namespace {
// Block-id range of the dK / dV grid: every id a base table can resolve.
int64_t ptr_bwd_blocks(int64_t max_base, int32_t blocks_per_chunk) {
  return blocks_per_chunk > 0 ? max_base * blocks_per_chunk : max_base;
}
}  // namespace

extern "C" size_t omm_sel_bwd_ptr_workspace_bytes(int64_t B, int64_t M, int64_t H,
                                                  int64_t max_base, int32_t blocks_per_chunk,
                                                  int32_t group_size, int64_t T,
                                                  int32_t compute_dkv) {
  if (B <= 0 || M <= 0 || H <= 0 || max_base < 0 || blocks_per_chunk < 0 || group_size < 1 || T < 1)
    return 0;
  const int64_t MG = omm::cdiv64(M, group_size);
  return omm::bwd_ws(B, M, H, MG, T, ptr_bwd_blocks(max_base, blocks_per_chunk), false,
                     compute_dkv != 0).total;
}

extern "C" int omm_sel_bwd_ptr(const omm_view4* q, const omm_view4* out, const float* lse,
                               const omm_view4* dout, const omm_view4* ids, const int64_t* ptr_k,
                               const int64_t* ptr_v, const int64_t* ptr_stride,
                               const int64_t* base_k, const int64_t* base_v,
                               const int64_t* base_dk, const int64_t* base_dv,
                               const int64_t* base_stride, int64_t max_base,
                               const int32_t* n_blocks_per_head, int32_t block_size,
                               int32_t group_size, int64_t batch_stride_kv_bytes,
                               int64_t batch_stride_dkv_bytes, int64_t stride_bn,
                               int64_t stride_bd, int64_t stride_dbn, int64_t stride_dbd,
                               int32_t blocks_per_chunk, int64_t in_chunk_block_bytes_kv,
                               int64_t in_chunk_block_bytes_dkv, float scale, int32_t compute_dkv,
                               const omm_view4* dq, float* delta, void* workspace,
                               size_t workspace_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE(q && out && lse && dout && ids && ptr_k && ptr_v && ptr_stride && dq && delta,
              OMM_EINVAL, "omm_sel_bwd_ptr: null argument");
  const int64_t B = q->size[0], M = q->size[1], H = q->size[2], D = q->size[3];
  for (int i = 0; i < 4; ++i)
    OMM_REQUIRE(out->size[i] == q->size[i] && dout->size[i] == q->size[i] &&
                    dq->size[i] == q->size[i],
                OMM_EINVAL, "omm_sel_bwd_ptr: out, d_out and dq must have q's shape");
  OMM_REQUIRE(group_size >= 1 && block_size >= 1, OMM_EINVAL,
              "omm_sel_bwd_ptr: group_size and block_size must be >= 1");
  const int64_t MG = cdiv64(M, group_size);
  OMM_REQUIRE(ids->size[0] == B && ids->size[1] == MG && ids->size[2] == H && ids->size[3] >= 1,
              OMM_EINVAL, "omm_sel_bwd_ptr: block_indices must be [%lld,%lld,%lld,T>=1]",
              (long long)B, (long long)MG, (long long)H);
  OMM_REQUIRE(stride_bn >= 0 && stride_bd >= 0, OMM_EINVAL, "omm_sel_bwd_ptr: negative stride");
  OMM_REQUIRE(D >= 1 && D <= 256, OMM_EUNSUPPORTED,
              "omm_sel_bwd_ptr: head dim must be in [1, 256] (got %lld)", (long long)D);
  OMM_REQUIRE(__builtin_isfinite(scale), OMM_EINVAL, "omm_sel_bwd_ptr: scale must be finite");
  const int64_t T = ids->size[3];
  const bool dkv = compute_dkv != 0;
  int64_t NS = 0;
  if (dkv) {
    OMM_REQUIRE(base_k && base_v && base_dk && base_dv && base_stride && max_base >= 0,
                OMM_EINVAL, "omm_sel_bwd_ptr: dK / dV need the four [H, max_base] base tables");
    OMM_REQUIRE(blocks_per_chunk >= 0, OMM_EINVAL, "omm_sel_bwd_ptr: blocks_per_chunk < 0");
    OMM_REQUIRE(blocks_per_chunk == 0 ||
                    (in_chunk_block_bytes_kv > 0 && in_chunk_block_bytes_dkv > 0),
                OMM_EINVAL, "omm_sel_bwd_ptr: chunk-level bases need in_chunk_block_bytes_kv/dkv > 0");
    OMM_REQUIRE(stride_dbn != 0 || D == 1, OMM_EINVAL,
                "omm_sel_bwd_ptr: stride_dbn must be the fp32 scratch row stride");
    NS = ptr_bwd_blocks(max_base, blocks_per_chunk);
  }
  OMM_REQUIRE(M <= 2147483647ll && MG * T <= 2147483647ll && B * H * MG * T <= 2147483647ll &&
                  NS <= 2147483647ll && B * H * (NS + 1) <= 2147483647ll,
              OMM_EUNSUPPORTED, "omm_sel_bwd_ptr: sizes exceed the int32 index range");
  if (B == 0 || M == 0 || H == 0) return OMM_OK;
  const BwdWs L = bwd_ws(B, M, H, MG, T, NS, false, dkv);
  OMM_REQUIRE(workspace != nullptr && workspace_bytes >= L.total &&
                  (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
              OMM_EWORKSPACE,
              "omm_sel_bwd_ptr: workspace of %zu bytes (256-byte aligned) required", L.total);
  PtrBwdArgs a;
  a.q = q;
  a.out = out;
  a.dout = dout;
  a.ids = ids;
  a.dq = dq;
  a.lse = lse;
  a.delta = delta;
  a.acc = PtrAcc{ptr_k, ptr_v, ptr_stride[0], ptr_stride[1], ptr_stride[2], ptr_stride[3],
                 stride_bn, block_size};
  a.kg = PtrGrad{base_k, base_v, base_dk, base_dv,
                 dkv ? base_stride[0] : 0, dkv ? base_stride[1] : 0, max_base, n_blocks_per_head,
                 batch_stride_kv_bytes, batch_stride_dkv_bytes, in_chunk_block_bytes_kv,
                 in_chunk_block_bytes_dkv, stride_bn, stride_bd, stride_dbn, stride_dbd,
                 blocks_per_chunk, block_size};
  a.bs = block_size;
  a.G = group_size;
  a.NS = static_cast<int>(NS);
  a.dkv = dkv;
  a.scale = scale;
  // MFMA kernels: head dim 64 / 128, unit dim stride and 16-byte row strides of the K / V blocks
  // (a block address itself may be 2-byte aligned), 16-byte q / out / d_out / dq rows and a
  // non-zero scale; everything else runs the VALU kernels
  bool rows_ok = true;
  for (const omm_view4* x : {q, out, dout, dq}) rows_ok = rows_ok && rows16(*x, D);
  const bool mfma = (D == 64 || D == 128) && stride_bd == 1 && stride_bn % 8 == 0 &&
                    2 * stride_bn * 64 < (int64_t{1} << 31) && rows_ok && scale != 0.0f;
  char* ws = static_cast<char*>(workspace);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (mfma) return D == 128 ? sel_bwd_ptr_launch<128, 0>(a, ws, L, s) : sel_bwd_ptr_launch<64, 0>(a, ws, L, s);
  if (D <= 64) return sel_bwd_ptr_launch<0, 16>(a, ws, L, s);
  if (D <= 128) return sel_bwd_ptr_launch<0, 32>(a, ws, L, s);
  return sel_bwd_ptr_launch<0, 64>(a, ws, L, s);
}
