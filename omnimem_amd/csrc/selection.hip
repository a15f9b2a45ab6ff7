// Selection attention forward: dense K/V, reference pointer tables, and the paged block cache.
//
// Reference semantics: cuda_backend/csrc/selection_fwd.cu:1-3 (fp32 softmax state, empty rows
// give O = 0 and LSE = -inf, natural-log LSE), common.cuh:158-215 (dense / pointer block
// resolution, partial blocks, pointer 0 = skip), :327-332 (chunk-causal visible prefix),
// selection_fwd.cu:218 (a query group's chunk is that of its first query).
//
// gfx950 design (bf16 / f16 queries): one workgroup = (b, query group of 64, head).
//   S^T = K Q^T on v_mfma_f32_16x16x32 (A = K rows from LDS, B = Q^T held in registers), so the
//   S^T accumulator already has the layout of the B operand of O^T = V^T P^T: P goes from the
//   softmax straight into the PV MFMA with no LDS round trip.
//   sel_fwd_dma_kernel (16-bit K / V): K / V tiles copied global -> LDS by buffer_load ... lds,
//   V read as V^T with ds_read_b64_tr_b16 (details at the kernel).
//   sel_fwd_mfma_kernel: register-staged variant for fp8 pages (e4m3 codes widened to bf16
//   while staging, page scales folded into the softmax) and for row strides the DMA kernel
//   cannot address.
// fp32 with 16-byte rows and head dim 64 or 128 runs sel_fwd_f32mfma_kernel (fp32 MFMA, split
// into equal runs per CU when the call has few items); any other shape a VALU kernel in full
// fp32.
#include <atomic>
#include <type_traits>

#include "sel_common.h"

namespace omm {
namespace {

// ---- staging: global -> registers -> LDS -----------------------------------------------------
// K tile in LDS: Ks[key][KP], KP = D + 8 (row pitch 272 B for D = 128: the 16-byte A-operand
// reads of 16 consecutive rows and the 16-byte row stores are both bank-conflict free).
// V tile in LDS, transposed: Vt[d][VP], VP = 72; the 4-key chunk c of row d is stored at chunk
// c ^ ((d >> 3) & 15), which makes both the transposing 8-byte stores (16 lanes: one key chunk,
// 16 row groups) and the 8-byte PV-operand reads (16 consecutive rows) conflict free.
constexpr int kVP = 72;


// Register staging of one 64-key tile by 128 threads.
//   K: unit u = tid + 128 j -> key tid / DC + (128 / DC) j, 8-dim slice tid % DC (DC lanes per row)
//   V: quad q = tid + 128 j -> dims slice tid % DC, keys 4 (tid / DC + (128 / DC) j) + r, r < 4
// Each thread's byte offset inside a tile is computed once; a tile adds a wave-uniform base, so
// the loads take the scalar-base + 32-bit-offset form with no per-load address arithmetic.
// fp8 pages (F8) keep the e4m3 codes in registers (8 bytes per unit) and widen them to bf16 only
// when the tile is stored to LDS (exact: every e4m3 value is a bf16 value).  The page scales are
// not applied here: the kernel folds them into the softmax (K's into the exponent scale, V's into
// p and the row sum), one per 64-key tile.  RAWK: K stays in codes in LDS too, for the fp8 QK^T
// MFMA.  NOK: K is not staged at all (the kernel copies it global -> LDS by DMA); only V is.
template <typename KVT, int D, bool RAWK = false, bool NOK = false>
struct Stager {
  static constexpr int DC = D / 8;                 // 16-byte slices per row
  static constexpr int KU = 64 * DC / 128;         // K units per thread
  static constexpr int VQ = 16 * DC / 128;         // V quads per thread
  static constexpr int RS = 128 / DC;              // rows between a thread's units
  static constexpr int ES = static_cast<int>(sizeof(KVT));
  static constexpr bool F8 = ES == 1;
  static constexpr int KP8 = D + 16;               // LDS row pitch of raw K codes (bytes)
  uint4 k[F8 || NOK ? 1 : KU];
  uint2 k8[F8 && !NOK ? KU : 1];
  uint4 v[F8 ? 1 : VQ][4];
  uint2 v8[F8 ? VQ : 1][4];
  uint32_t koff, voff;                             // bytes, within a tile

  __device__ __forceinline__ void init(int tid, int64_t sk, int64_t sv) {
    koff = static_cast<uint32_t>(((tid / DC) * sk + (tid % DC) * 8) * ES);
    voff = static_cast<uint32_t>((4 * (tid / DC) * sv + (tid % DC) * 8) * ES);
  }

  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int j = 0; j < (NOK ? 0 : KU); ++j) {
      if constexpr (F8) k8[j] = make_uint2(0, 0);
      else k[j] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < VQ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (F8) v8[j][r] = make_uint2(0, 0);
        else v[j][r] = make_uint4(0, 0, 0, 0);
      }
  }

  // Rows at or past n are not loaded: their registers keep finite values from an earlier tile
  // (or the initial zeros).  Their scores are masked to -inf, so their V rows get weight 0.
  // MIS: the accessor admits blocks that are not 16-byte aligned (raw pointer tables); such a
  // block is read with 2-byte loads (wave-uniform test on the block's addresses).
  template <bool MIS = false>
  __device__ __forceinline__ void load(const BlockRef& br, int tok0, int n, int tid) {
    if constexpr (MIS) {
      if (((reinterpret_cast<uintptr_t>(br.k) | reinterpret_cast<uintptr_t>(br.v)) & 15u) != 0u) {
        load_impl<false, true>(br, tok0, n, tid);
        return;
      }
    }
    if (n >= 64)
      load_impl<true>(br, tok0, n, tid);
    else
      load_impl<false>(br, tok0, n, tid);
  }

  __device__ __forceinline__ static uint4 load_u16(const char* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    uint32_t wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      wd[i] = static_cast<uint32_t>(h[2 * i]) | (static_cast<uint32_t>(h[2 * i + 1]) << 16);
    return make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }

  template <bool FULL, bool U16 = false>
  __device__ __forceinline__ void load_impl(const BlockRef& br, int tok0, int n, int tid) {
    const char* kb = static_cast<const char*>(br.k) + static_cast<int64_t>(tok0) * br.sk * ES;
    const char* vb = static_cast<const char*>(br.v) + static_cast<int64_t>(tok0) * br.sv * ES;
    const int row0 = tid / DC;
#pragma unroll
    for (int j = 0; j < (NOK ? 0 : KU); ++j) {
      const char* p = kb + static_cast<int64_t>(RS * j) * br.sk * ES;
      if (FULL || row0 + RS * j < n) {
        if constexpr (F8) k8[j] = *reinterpret_cast<const uint2*>(p + koff);
        else if constexpr (U16) k[j] = load_u16(p + koff);
        else k[j] = *reinterpret_cast<const uint4*>(p + koff);
      }
    }
#pragma unroll
    for (int j = 0; j < VQ; ++j) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const char* p = vb + static_cast<int64_t>(4 * RS * j + r) * br.sv * ES;
        if (FULL || 4 * (row0 + RS * j) + r < n) {
          if constexpr (F8) v8[j][r] = *reinterpret_cast<const uint2*>(p + voff);
          else if constexpr (U16) v[j][r] = load_u16(p + voff);
          else v[j][r] = *reinterpret_cast<const uint4*>(p + voff);
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* Ks, uint16_t* Vt, int tid) const {
    constexpr int KP = D + 8;
    const int dc = tid % DC;
#pragma unroll
    for (int j = 0; j < (NOK ? 0 : KU); ++j) {
      const int key = tid / DC + RS * j;
      if constexpr (RAWK)
        *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(Ks) + key * KP8 + dc * 8) = k8[j];
      else if constexpr (F8)
        *reinterpret_cast<uint4*>(Ks + key * KP + dc * 8) = e4m3x8_to_bf16(k8[j]);
      else
        *reinterpret_cast<uint4*>(Ks + key * KP + dc * 8) = k[j];
    }
#pragma unroll
    for (int j = 0; j < VQ; ++j) {
      const int kq = tid / DC + RS * j;
      uint4 vr4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (F8) vr4[r] = e4m3x8_to_bf16(v8[j][r]);
        else vr4[r] = v[j][r];
      }
      const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&vr4[0]);
      const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&vr4[1]);
      const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&vr4[2]);
      const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&vr4[3]);
      // rows 8 dc .. 8 dc + 7 share the swizzle (8 dc) >> 3 = dc
      uint16_t* vrow = Vt + (8 * dc) * kVP + ((kq ^ (dc & 15)) << 2);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // dims 8dc + 2e (low halves) and 8dc + 2e + 1 (high halves) of the 4 keys
        const uint2 lo = make_uint2(__builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u),
                                    __builtin_amdgcn_perm(w3[e], w2[e], 0x05040100u));
        const uint2 hi = make_uint2(__builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u),
                                    __builtin_amdgcn_perm(w3[e], w2[e], 0x07060302u));
        *reinterpret_cast<uint2*>(vrow + (2 * e) * kVP) = lo;
        *reinterpret_cast<uint2*>(vrow + (2 * e + 1) * kVP) = hi;
      }
    }
  }
};

// ---- MFMA kernel ------------------------------------------------------------------------------
// One workgroup = (b, head, 64 queries of one query group), 2 waves x 32 queries.  Each wave owns
// two 16-query MFMA row blocks that share every K and V^T operand read from LDS, so the LDS
// bytes per MFMA FLOP are half those of 16 queries per wave.
constexpr int kMfmaThreads = 128;

// QK8 (fp8 pages only): the queries are quantised to e4m3 per query row (scale amax / 448), K
// stays in its page codes, S = (Qc Kc^T) * s_q * s_k on v_mfma_f32_16x16x32_fp8_fp8 (products
// of e4m3 codes are exact in fp32), the K page scale s_k is one per 64-key tile and s_q one per
// query column, both folded into the softmax's exponent scale.  PV stays bf16.
// At D = 128 the K codes need no widening, so they skip the registers: each tile's 64 rows of 128
// bytes go global -> LDS by buffer_load ... lds (4 instructions per wave) into one of two 8 KiB
// buffers, issued a tile ahead like the register loads of V.  16-byte chunk c of row r sits at
// slot c ^ kSwz8(r), which keeps the b128 operand reads conflict free whether a read cycle
// serves 8 lanes (32 banks) or 16 (64 banks).  One b128 read feeds two fp8 k-steps: k-step s of
// lane group j4 covers head dims 64 (s >> 1) + 16 j4 + 8 (s & 1) .. +7 for K and for Q alike.
__device__ __forceinline__ int kSwz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <typename QT, typename Acc, int D, bool QK8 = false>
__global__ __launch_bounds__(kMfmaThreads, 2) void sel_fwd_mfma_kernel(
    View4<const QT> q, View4<QT> out, float* __restrict__ lse, Acc acc, int M, int H, int G,
    int MG, int T, int chunk, float scale, int nsub) {
  constexpr int KP = D + 8;
  constexpr int KS = 64 * KP, VS = D * kVP;
  constexpr int SD = D / 32;   // k-steps of QK^T
  constexpr int ND = D / 16;   // d-tiles of PV
  static_assert(!QK8 || sizeof(typename Acc::KV) == 1, "fp8 QK^T needs fp8 pages");
  constexpr bool DMAK = QK8 && D == 128;  // K codes by LDS DMA (two 8 KiB buffers in Ks)
  static_assert(!DMAK || 2 * 8192 <= KS * 2, "K DMA buffers fit the K region");
  __shared__ __align__(16) uint16_t lds[KS + VS];
  uint16_t* Ks = lds;
  uint16_t* Vt = lds + KS;

  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
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
  if (sub == 0) acc.touch(b, g, h, T);

  // Q^T operands of this wave's two 16-query blocks: row my_q[qb], dims 32 s + 8 j4 .. +7
  int my_q[2];
  bool q_ok[2];
  uint4 qb[2][SD];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    my_q[x] = m0 + 32 * w + 16 * x + l16;
    q_ok[x] = my_q[x] < m_end;
#pragma unroll
    for (int s = 0; s < SD; ++s) {
      const int d0 = DMAK ? 64 * (s >> 1) + 16 * j4 + 8 * (s & 1) : 32 * s + 8 * j4;
      qb[x][s] = q_ok[x] ? *reinterpret_cast<const uint4*>(q.at(b, my_q[x], h, d0))
                         : make_uint4(0, 0, 0, 0);
    }
  }
  // fp8 queries: per-row amax over the 4 lane groups holding the row's dims, scale amax / 448,
  // codes by round-to-nearest-even (v_cvt_pk_fp8_f32)
  uint2 qb8[2][SD];
  float sq[2] = {1.0f, 1.0f};
  if constexpr (QK8) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      float f[SD][8];
      float am = 0.0f;
#pragma unroll
      for (int s = 0; s < SD; ++s) {
        unpack_bf16x8_sel(qb[x][s], f[s]);
#pragma unroll
        for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(f[s][e]));
      }
      am = fmaxf(am, __shfl_xor(am, 16, kWave));
      am = fmaxf(am, __shfl_xor(am, 32, kWave));
      sq[x] = am > 0.0f ? am / 448.0f : 1.0f;
      const float inv = am > 0.0f ? 448.0f / am : 1.0f;
#pragma unroll
      for (int s = 0; s < SD; ++s) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = fminf(fmaxf(f[s][e] * inv, -448.0f), 448.0f);
        qb8[x][s] = make_uint2(f32x4_to_e4m3(y[0], y[1], y[2], y[3]),
                               f32x4_to_e4m3(y[4], y[5], y[6], y[7]));
      }
    }
  }
  const bool wave_active = (m0 + 32 * w) < m_end;
  // PV operand row bases (see the V^T swizzle): bit 0 of the chunk is j4_0 ^ (l16 >> 3), bit 1
  // is j4_1 ^ (i & 1)
  const int sw0 = (j4 & 1) ^ (l16 >> 3);
  const uint16_t* vb[2] = {Vt + l16 * kVP + 4 * sw0 + 8 * (j4 >> 1),
                           Vt + l16 * kVP + 4 * sw0 + 8 * (1 - (j4 >> 1))};

  f32x4 o[2][ND];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int i = 0; i < ND; ++i) o[x][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m2[2] = {kNegInf, kNegInf}, lsum[2] = {0.0f, 0.0f};
  bool started = false;  // every row of the wave has seen a visible key (kLazyMax)
  // the softmax works on s * c2 with c2 > 0; a negative scale negates Q instead, which is exact
  // (the host routes a zero or non-finite scale to the VALU kernel)
  float c2 = scale * kLog2e;
  if (c2 < 0.0f) {
    c2 = -c2;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int s = 0; s < SD; ++s) {
        qb[x][s].x ^= 0x80008000u;
        qb[x][s].y ^= 0x80008000u;
        qb[x][s].z ^= 0x80008000u;
        qb[x][s].w ^= 0x80008000u;
        qb8[x][s].x ^= 0x80808080u;  // e4m3 sign bits
        qb8[x][s].y ^= 0x80808080u;
      }
  }

  using KVT = typename Acc::KV;
  constexpr bool kFp8 = sizeof(KVT) == 1;
  // fp8 pages at D = 128 take the running max only when it must move (below); the other
  // instances keep a per-tile max test, which needs fewer registers
  constexpr bool kLazyMax = kFp8 && D == 128;
  Stager<KVT, D, QK8, DMAK> st;
  float sk_next = 1.0f, sv_next = 1.0f;  // page scales of the tile being staged (fp8 pages)
  WaveWalk<Acc> wk;
  wk.start(acc, b, g, h, T, qc);
  st.init(tid, wk.br.sk, wk.br.sv);  // row strides are the same for every block of a call
  st.zero();
  // raw pointer tables may hold blocks that are not 16-byte aligned (2-byte loads for those)
  constexpr bool kMis = Acc::kMayMisalign && sizeof(KVT) == 2;
  // DMAK: this lane's source offsets for the wave's 4 copy instructions (rows 32 w .. 32 w + 31)
  // and its operand read offsets (row l16, chunk 4 p + j4; the 16 t rows are an immediate)
  int kdo[4] = {0, 0, 0, 0}, k8off[2] = {0, 0};
  int rsk = 0, kbi = 0;
  char* const kbuf = reinterpret_cast<char*>(Ks);
  if constexpr (DMAK) {
#pragma unroll
    for (int p = 0; p < 2; ++p) k8off[p] = l16 * D + (((4 * p + j4) ^ kSwz8(l16)) << 4);
  }
  if (wk.valid) {
    if constexpr (DMAK) {
      rsk = static_cast<int>(wk.br.sk);  // bytes: one code per element
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int row = (4 * w + jj) * 8 + lane / 8, c = lane % 8;
        kdo[jj] = row * rsk + ((c ^ kSwz8(row)) << 4);
      }
      dma_part<4>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(wk.tok0) * rsk, rsk,
                  wk.n, kbuf, w, kdo);
    }
    st.template load<kMis>(wk.br, wk.tok0, wk.n, tid);
    if constexpr (kFp8) {
      sk_next = wk.br.scale_k;
      sv_next = wk.br.scale_v;
    }
  }
  while (wk.valid) {
    // this wave's K copy of the tile has landed (DMAK); after the barrier every wave's has, and
    // every wave is done reading the previous tile
    if constexpr (DMAK) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    st.store(Ks, Vt, tid);
    __syncthreads();
    const int tile_n = wk.n;
    const float sk_cur = sk_next, sv_cur = sv_next;
    const char* const kcur = kbuf + 8192 * kbi;
    wk.advance(acc, b, g, h, T, qc);
    if (wk.valid) {
      if constexpr (DMAK)  // into the other buffer, which every wave finished reading last tile
        dma_part<4>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(wk.tok0) * rsk, rsk,
                    wk.n, kbuf + 8192 * (kbi ^ 1), w, kdo);
      st.template load<kMis>(wk.br, wk.tok0, wk.n, tid);  // in flight during the MFMAs
      if constexpr (kFp8) {
        sk_next = wk.br.scale_k;
        sv_next = wk.br.scale_v;
      }
    }
    // exponent scale per query block: the softmax scale, for fp8 pages times the K page scale
    // (and the query scale of fp8 scores).  V's page scale goes into p as 2^(log2 s_v): p s_v
    // feeds the PV MFMA and the row sum takes the tile's sum divided by s_v.
    float c2x[2] = {c2, c2};
    float lv = 0.0f, inv_sv = 1.0f;
    if constexpr (QK8) {
      c2x[0] = c2 * sq[0] * sk_cur;
      c2x[1] = c2 * sq[1] * sk_cur;
    } else if constexpr (kFp8) {
      c2x[0] = c2x[1] = c2 * sk_cur;
    }
    if constexpr (kFp8) {
      lv = __builtin_amdgcn_logf(sv_cur);     // log2 (scales are normal floats)
      inv_sv = __builtin_amdgcn_rcpf(sv_cur);
    }
    if (wave_active) {
      // S^T = K Q^T: lane holds keys 16 t + 4 j4 + r of query l16, for both query blocks.  A
      // partial tile seeds the accumulators with 0 / -inf per key, so masked keys come out -inf.
      f32x4 s4[2][4];
      if (tile_n >= 64) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          s4[0][t] = f32x4{0.f, 0.f, 0.f, 0.f};
          s4[1][t] = f32x4{0.f, 0.f, 0.f, 0.f};
          if constexpr (DMAK) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              const uint4 a = *reinterpret_cast<const uint4*>(kcur + k8off[p] + 16 * D * t);
              s4[0][t] = mfma_fp8(make_uint2(a.x, a.y), qb8[0][2 * p], s4[0][t]);
              s4[1][t] = mfma_fp8(make_uint2(a.x, a.y), qb8[1][2 * p], s4[1][t]);
              s4[0][t] = mfma_fp8(make_uint2(a.z, a.w), qb8[0][2 * p + 1], s4[0][t]);
              s4[1][t] = mfma_fp8(make_uint2(a.z, a.w), qb8[1][2 * p + 1], s4[1][t]);
            }
          } else
#pragma unroll
          for (int s = 0; s < SD; ++s) {
            if constexpr (QK8) {
              const uint2 a8 = *reinterpret_cast<const uint2*>(
                  reinterpret_cast<const uint8_t*>(Ks) + (16 * t + l16) * Stager<KVT, D, true>::KP8 +
                  32 * s + 8 * j4);
              s4[0][t] = mfma_fp8(a8, qb8[0][s], s4[0][t]);
              s4[1][t] = mfma_fp8(a8, qb8[1][s], s4[1][t]);
            } else {
              const uint4 a = *reinterpret_cast<const uint4*>(Ks + (16 * t + l16) * KP + 32 * s + 8 * j4);
              s4[0][t] = Mfma<QT>::run(a, qb[0][s], s4[0][t]);
              s4[1][t] = Mfma<QT>::run(a, qb[1][s], s4[1][t]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);  // bound the operand reads in flight (registers)
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int lim = tile_n - 16 * t - 4 * j4;
          const f32x4 bias{lim > 0 ? 0.f : kNegInf, lim > 1 ? 0.f : kNegInf,
                           lim > 2 ? 0.f : kNegInf, lim > 3 ? 0.f : kNegInf};
          s4[0][t] = bias;
          s4[1][t] = bias;
          if constexpr (DMAK) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              const uint4 a = *reinterpret_cast<const uint4*>(kcur + k8off[p] + 16 * D * t);
              s4[0][t] = mfma_fp8(make_uint2(a.x, a.y), qb8[0][2 * p], s4[0][t]);
              s4[1][t] = mfma_fp8(make_uint2(a.x, a.y), qb8[1][2 * p], s4[1][t]);
              s4[0][t] = mfma_fp8(make_uint2(a.z, a.w), qb8[0][2 * p + 1], s4[0][t]);
              s4[1][t] = mfma_fp8(make_uint2(a.z, a.w), qb8[1][2 * p + 1], s4[1][t]);
            }
          } else
#pragma unroll
          for (int s = 0; s < SD; ++s) {
            if constexpr (QK8) {
              const uint2 a8 = *reinterpret_cast<const uint2*>(
                  reinterpret_cast<const uint8_t*>(Ks) + (16 * t + l16) * Stager<KVT, D, true>::KP8 +
                  32 * s + 8 * j4);
              s4[0][t] = mfma_fp8(a8, qb8[0][s], s4[0][t]);
              s4[1][t] = mfma_fp8(a8, qb8[1][s], s4[1][t]);
            } else {
              const uint4 a = *reinterpret_cast<const uint4*>(Ks + (16 * t + l16) * KP + 32 * s + 8 * j4);
              s4[0][t] = Mfma<QT>::run(a, qb[0][s], s4[0][t]);
              s4[1][t] = Mfma<QT>::run(a, qb[1][s], s4[1][t]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // P^T operands (k-slot e of lane group j4 is key 32 u + 4 j4 + e, e < 4, or 32 u + 16 +
      // 4 j4 + (e - 4))
      uint4 pb[2][2];
      if constexpr (kLazyMax) {
        // online softmax in the log2 domain: e = s c2x - msafe (plus log2 s_v for fp8 pages),
        // p = 2^e, msafe = m2 (0 while m2 = -inf), shared by the 4 lane groups of a query.  m2
        // (the largest s c2x seen when it last moved) moves before a row's first visible key
        // and when some lane's sum of the tile's p / s_v for the row passes 256; a move
        // recomputes the tile's p.  So the common path takes no max, p stays small, and a move
        // gives the new largest key p = 1.
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const float bias = (kFp8 ? lv : 0.0f) - (m2[x] == kNegInf ? 0.0f : m2[x]);
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) s4[x][t][r] = __builtin_fmaf(s4[x][t][r], c2x[x], bias);
        }
        auto move_max = [&]() {
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            const float msafe = m2[x] == kNegInf ? 0.0f : m2[x];
            float v = kNegInf;
#pragma unroll
            for (int t = 0; t < 4; ++t)
              v = fmaxf(v, fmaxf(fmaxf(s4[x][t][0], s4[x][t][1]), fmaxf(s4[x][t][2], s4[x][t][3])));
            v = fmaxf(v, __shfl_xor(v, 16, kWave));
            v = fmaxf(v, __shfl_xor(v, 32, kWave));
            // v: the query's largest e of this tile, relative to msafe (and log2 s_v)
            const float mcand = fmaxf(m2[x], (kFp8 ? v - lv : v) + msafe);
            const float msafe_new = mcand == kNegInf ? 0.0f : mcand;
            const float alpha = __builtin_amdgcn_exp2f(m2[x] - msafe_new);
            lsum[x] *= alpha;
#pragma unroll
            for (int i = 0; i < ND; ++i) o[x][i] *= alpha;
            m2[x] = mcand;
            const float shift = msafe - msafe_new;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
              for (int r = 0; r < 4; ++r) s4[x][t][r] += shift;
          }
        };
        if (!started) {  // wave-uniform: some row has not seen a visible key yet
          move_max();
          started = __ballot(m2[0] == kNegInf || m2[1] == kNegInf) == 0ull;
        }
        float ps[2];  // the lane's sum of the tile's p per row (times s_v for fp8 pages)
        auto exps = [&]() {
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            float pv[4][4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
              for (int r = 0; r < 4; ++r) pv[t][r] = __builtin_amdgcn_exp2f(s4[x][t][r]);
            // the first group's sum starts ps (0 + x is not folded: it would turn -0 into +0)
            float sum = (pv[0][0] + pv[0][1]) + (pv[0][2] + pv[0][3]);
#pragma unroll
            for (int t = 1; t < 4; ++t) sum += (pv[t][0] + pv[t][1]) + (pv[t][2] + pv[t][3]);
            ps[x] = sum;
#pragma unroll
            for (int u = 0; u < 2; ++u)
              pb[u][x] = make_uint4(Mfma<QT>::pack2(pv[2 * u][0], pv[2 * u][1]),
                                    Mfma<QT>::pack2(pv[2 * u][2], pv[2 * u][3]),
                                    Mfma<QT>::pack2(pv[2 * u + 1][0], pv[2 * u + 1][1]),
                                    Mfma<QT>::pack2(pv[2 * u + 1][2], pv[2 * u + 1][3]));
          }
        };
        exps();
        const float bound = kFp8 ? 256.0f * sv_cur : 256.0f;  // 256 for p / s_v
        if (__ballot(ps[0] > bound || ps[1] > bound) != 0ull) {
          move_max();
          exps();
        }
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          if constexpr (kFp8) lsum[x] = __builtin_fmaf(ps[x], inv_sv, lsum[x]);
          else lsum[x] += ps[x];
        }
      } else {
        // online softmax in the log2 domain: p = 2^(s * c2 - m), m a running max of s * c2 shared
        // by the 4 lane groups of a query.  m is raised only when some lane's tile max exceeds it
        // by more than 2^8 (p then stays <= 256, exact enough in fp32 and in the bf16 P operand),
        // so after the first tiles the cross-lane max reduction is rarely needed.
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          float mt = kNegInf;
#pragma unroll
          for (int t = 0; t < 4; ++t)
            mt = fmaxf(mt, fmaxf(fmaxf(s4[x][t][0], s4[x][t][1]), fmaxf(s4[x][t][2], s4[x][t][3])));
          if (__ballot(mt * c2x[x] > m2[x] + 8.0f) != 0ull) {
            mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
            mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
            const float mcand = fmaxf(m2[x], mt * c2x[x]);
            const float msafe_new = mcand == kNegInf ? 0.0f : mcand;
            const float alpha = __builtin_amdgcn_exp2f(m2[x] - msafe_new);
            lsum[x] *= alpha;
#pragma unroll
            for (int i = 0; i < ND; ++i) o[x][i] *= alpha;
            m2[x] = mcand;
          }
          const float msafe = m2[x] == kNegInf ? 0.0f : m2[x];
          const float bias = kFp8 ? lv - msafe : -msafe;
          float ps = 0.0f;
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s4[x][t][r], c2x[x], bias));
              s4[x][t][r] = pv;
              ps += pv;
            }
          if constexpr (kFp8) lsum[x] = __builtin_fmaf(ps, inv_sv, lsum[x]);
          else lsum[x] += ps;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int x = 0; x < 2; ++x)
            pb[u][x] = make_uint4(Mfma<QT>::pack2(s4[x][2 * u][0], s4[x][2 * u][1]),
                                  Mfma<QT>::pack2(s4[x][2 * u][2], s4[x][2 * u][3]),
                                  Mfma<QT>::pack2(s4[x][2 * u + 1][0], s4[x][2 * u + 1][1]),
                                  Mfma<QT>::pack2(s4[x][2 * u + 1][2], s4[x][2 * u + 1][3]));
      }
      // O^T += V^T P^T; k-slot e of lane group j4 is key 32u + 4 j4 + e (e < 4) or
      // 32u + 16 + 4 j4 + (e - 4), for both operands
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int i = 0; i < ND; ++i) {
          // row d = 16i + l16, chunk c = 8u + 4h + j4 stored at c ^ (2i + (l16 >> 3)): the
          // lane-dependent bits are in vb[i & 1], the rest is a compile-time offset
          const int i1 = (i >> 1) & 1, i2 = (i >> 2) & 1;
          const uint16_t* vr = vb[i & 1] + (16 * i) * kVP + 32 * (u ^ i2);
          const uint2 lo = *reinterpret_cast<const uint2*>(vr + 16 * i1);
          const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16 * (1 - i1));
          const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
          o[0][i] = Mfma<QT>::run(a, pb[u][0], o[0][i]);
          o[1][i] = Mfma<QT>::run(a, pb[u][1], o[1][i]);
          if ((i & 1) == 1) __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    kbi ^= 1;
  }

  // epilogue: reduce the lane-partial sums of each query over its 4 lane groups
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    float ls = lsum[x];
    ls += __shfl_xor(ls, 16, kWave);
    ls += __shfl_xor(ls, 32, kWave);
    if (q_ok[x]) {
      const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
      QT* op = out.at(b, my_q[x], h, 0);
#pragma unroll
      for (int i = 0; i < ND; ++i) {
        const int d0 = 16 * i + 4 * j4;
        uint2 w2;
        w2.x = Mfma<QT>::pack2(o[x][i][0] * inv, o[x][i][1] * inv);
        w2.y = Mfma<QT>::pack2(o[x][i][2] * inv, o[x][i][3] * inv);
        *reinterpret_cast<uint2*>(op + d0) = w2;
      }
      if (lse != nullptr && j4 == 0)
        lse[(static_cast<int64_t>(b) * H + h) * M + my_q[x]] =
            ls > 0.0f ? (m2[x] + __builtin_log2f(ls)) * kLn2 : kNegInf;
    }
  }
}

// ---- DMA kernel (16-bit K / V) ----------------------------------------------------------------
// One workgroup = up to 64 queries of one query group (NW = 2 waves) or two 64-query subgroups
// of one group (NW = 4); each wave owns 32 queries (2 MFMA row blocks of 16 each, sharing every
// K and V^T operand read), 2 waves per SIMD.  K and V tiles of TK keys (8 KiB each) go
// global -> LDS by buffer_load ... lds with no register staging; rows past the block's visible
// tokens read as 0 through the buffer bound, so a partial tile holds finite values.  Two LDS
// buffers each for K and V: the copy of tile i + 1 is issued right after the barrier that opens
// tile i (each wave issues 8 / NW of a tile's copy instructions and waits for its own before
// that barrier).
//   LDS K rows:  16-byte chunk c of row r at slot c ^ (r % CPR), so the 16-row b128 operand reads
//                of one chunk column hit 16 distinct slots;
//   LDS V rows:  chunk c of row r at slot c ^ (2 (r % 8) % CPR); the V^T operand comes from
//                ds_read_b64_tr_b16, which gives lane L of a 16-lane group element L of the 4
//                rows its group addresses: 4 consecutive keys of one head dim.

// NW = 4 serves query groups of more than 64 queries: the 4 waves share every K / V tile, which
// halves the copies per query.
template <typename QT, typename Acc, int D, int NW>
__global__ __launch_bounds__(NW * kWave, 2) void sel_fwd_dma_kernel(
    View4<const QT> q, View4<QT> out, float* __restrict__ lse, Acc acc, int M, int H, int G,
    int MG, int T, int chunk, float scale, int nsub, GateArgs gate) {
  static_assert(NW == 2 || NW == 4, "2 or 4 waves");
  constexpr int SPW = NW / 2;  // 64-query subgroups per workgroup
  constexpr int NI = 8 / NW;   // copy instructions per wave per K or V tile
  using DG = DmaGeom<D>;
  constexpr int ROWB = DG::ROWB, CPR = DG::CPR, TK = DG::TK, RPI = DG::RPI;
  constexpr int NT = DG::NT, NU = DG::NU, SD = DG::SD, ND = DG::ND;
  __shared__ __align__(16) char lds[4][8192];  // K buffers 0, 1; V buffers 2, 3

  const int tid = static_cast<int>(threadIdx.x), lane = lane_id(), w = tid / kWave;
  const int l16 = lane & 15, j4 = lane >> 4;
  const int total = static_cast<int>(gridDim.x);
  const int nsw = (nsub + SPW - 1) / SPW;  // workgroups per query group
  int wi = xcd_remap(static_cast<int>(blockIdx.x), total);
  const int sw = wi % nsw; wi /= nsw;
  const int g = wi % MG; wi /= MG;
  const int h = wi % H;
  const int b = wi / H;

  // this wave's 32 queries: subgroup sub, half ws (a subgroup past the group has none)
  const int sub = sw * SPW + w / 2, ws = w & 1;
  const int m0 = g * G + sub * 64;
  const int m_end = min(min(g * G + G, M), m0 + 64);
  const int qc = (g * G) / chunk;
  if (sw == 0) acc.touch(b, g, h, T);

  // Q^T operands of this wave's 2 query blocks: row m0 + 32 ws + 16 x + l16, dims 32 s + 8 j4 ..
  bool q_ok[2];
  uint4 qb[2][SD];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int mq = m0 + 32 * ws + 16 * x + l16;
    q_ok[x] = mq < m_end;
#pragma unroll
    for (int s = 0; s < SD; ++s)
      qb[x][s] = q_ok[x] ? *reinterpret_cast<const uint4*>(q.at(b, mq, h, 32 * s + 8 * j4))
                         : make_uint4(0, 0, 0, 0);
  }
  // the softmax works on s * c2 with c2 > 0; a negative scale negates Q instead, which is exact
  float c2 = scale * kLog2e;
  if (c2 < 0.0f) {
    c2 = -c2;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int s = 0; s < SD; ++s) {
        qb[x][s].x ^= 0x80008000u;
        qb[x][s].y ^= 0x80008000u;
        qb[x][s].z ^= 0x80008000u;
        qb[x][s].w ^= 0x80008000u;
      }
  }

  // LDS read offsets inside a tile buffer.  K operand (t, s): row 16 t + l16, chunk 4 s + j4
  // (16 t rows are a compile-time offset).  V^T operand (u, half, i): row 32 u + 16 half + 4 j4
  // + (l16 >> 2), dims 16 i + 4 (l16 & 3) .. +3.
  int koff[SD], voff[ND];
#pragma unroll
  for (int s = 0; s < SD; ++s) koff[s] = l16 * ROWB + (((4 * s + j4) ^ DG::swz_k(l16)) << 4);
  {
    const int vr = 4 * j4 + (l16 >> 2), vm = l16 & 3;
#pragma unroll
    for (int i = 0; i < ND; ++i)
      voff[i] = vr * ROWB + (((2 * i + (vm >> 1)) ^ DG::swz_v(vr)) << 4) + ((vm & 1) << 3);
  }

  f32x4 o[2][ND];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int i = 0; i < ND; ++i) o[x][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m2[2] = {kNegInf, kNegInf};
  float nms[2] = {0.0f, 0.0f};  // -max(m2, 0 if none finite)
  float lsum[2] = {0.0f, 0.0f};  // fp32 row sums of the unrounded p (lane partials)
  bool started = false;          // every row of the wave has seen a visible key

  WaveWalk<Acc, TK> wk;
  wk.start(acc, b, g, h, T, qc);
  int n_cur = 0;        // visible keys of the current tile (0: done)
  int kdo[NI], vdo[NI];  // this lane's source offsets of this wave's copy instructions
  int rsk = 0, rsv = 0;
  if (wk.valid) {
    // row strides are the same for every block of a call
    rsk = static_cast<int>(wk.br.sk) * 2;
    rsv = static_cast<int>(wk.br.sv) * 2;
#pragma unroll
    for (int jj = 0; jj < NI; ++jj) {
      const int row = (NI * w + jj) * RPI + lane / CPR, c = lane % CPR;
      kdo[jj] = row * rsk + ((c ^ DG::swz_k(row)) << 4);
      vdo[jj] = row * rsv + ((c ^ DG::swz_v(row)) << 4);
    }
    copy_part<Acc>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(wk.tok0) * rsk, rsk, wk.n,
             lds[0], w, kdo);
    copy_part<Acc>(static_cast<const char*>(wk.br.v) + static_cast<int64_t>(wk.tok0) * rsv, rsv, wk.n,
             lds[2], w, vdo);
    n_cur = wk.n;
    wk.advance(acc, b, g, h, T, qc);
  }

  // Q and the block walk's loads are complete before the loop: without this compiler-visible
  // wait the loop would re-wait vmcnt(0) every tile (for loads it cannot tell are done), which
  // would also wait for the next tile's copy.
  __builtin_amdgcn_s_waitcnt(0);

  // One key tile in LDS buffers BI (0 or 1), a compile-time constant so that every LDS address
  // is a lane offset plus an immediate.
  auto step = [&](auto BIc) -> bool {
    constexpr int BI = decltype(BIc)::value;
    // this wave's copies of the tile are in LDS; after the barrier every wave's are, and every
    // wave is done reading buffers BI ^ 1 (the previous tile)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int n_nx = 0;
    if (wk.valid) {
      const int tok = __builtin_amdgcn_readfirstlane(wk.tok0);  // uniform: scalar arithmetic
      copy_part<Acc>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(tok) * rsk, rsk,
               wk.n, lds[BI ^ 1], w, kdo);
      copy_part<Acc>(static_cast<const char*>(wk.br.v) + static_cast<int64_t>(tok) * rsv, rsv,
               wk.n, lds[2 + (BI ^ 1)], w, vdo);
      n_nx = wk.n;
      wk.advance(acc, b, g, h, T, qc);
    }
    const char* Kt = lds[BI];
    const char* Vt = lds[2 + BI];

    // S^T = K Q^T: lane holds keys 16 t + 4 j4 + r of query l16, for both query blocks.  All K
    // operand reads are issued before the first MFMA, and all V^T operand reads right after the
    // last one, so that their LDS latency overlaps the MFMAs and the softmax instead of
    // stalling each MFMA pair on its own read.
    uint4 ka[NT][SD];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int s = 0; s < SD; ++s)
        ka[t][s] = *reinterpret_cast<const uint4*>(Kt + koff[s] + 16 * t * ROWB);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 s4[2][NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      s4[0][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      s4[1][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < SD; ++s) {
        s4[0][t] = Mfma<QT>::run(ka[t][s], qb[0][s], s4[0][t]);
        s4[1][t] = Mfma<QT>::run(ka[t][s], qb[1][s], s4[1][t]);
      }
    }
    uint4 va[NU][ND];
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int i2 = 0; i2 < ND; ++i2) {
        const uint2 lo = lds_read_tr16(Vt + voff[i2] + (32 * u) * ROWB);
        const uint2 hi = lds_read_tr16(Vt + voff[i2] + (32 * u + 16) * ROWB);
        va[u][i2] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
    __builtin_amdgcn_sched_barrier(0);
    if (n_cur < TK) {  // partial tile: keys past n_cur are not visible
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (16 * t + 4 * j4 + r >= n_cur) s4[0][t][r] = s4[1][t][r] = kNegInf;
    }

    // online softmax in the log2 domain: e = s c2 - msafe per query, p = 2^e, msafe = m2 (0
    // while m2 = -inf).  m2 (the largest s c2 seen when it last moved) moves before a row's first
    // visible key and when some lane's sum of the tile's p for the row passes 256, so the common
    // path takes no max at all.  The bound keeps p small, and a move makes the new largest key's
    // p exactly 1: with a bound of 2^60 instead, peaked rows (scale 8) lost accuracy to the
    // rounding of their dominant p to 16 bits (simulated mean error 1.12e-3 against 0.99e-3).
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const float msafe = -nms[x];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) s4[x][t][r] = __builtin_fmaf(s4[x][t][r], c2, -msafe);
    }
    auto move_max = [&]() {
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const float msafe = m2[x] == kNegInf ? 0.0f : m2[x];
        float v = kNegInf;
#pragma unroll
        for (int t = 0; t < NT; ++t)
          v = fmaxf(v, fmaxf(fmaxf(s4[x][t][0], s4[x][t][1]), fmaxf(s4[x][t][2], s4[x][t][3])));
        v = fmaxf(v, __shfl_xor(v, 16, kWave));
        v = fmaxf(v, __shfl_xor(v, 32, kWave));
        // v: the query's largest e of this tile, relative to msafe
        const float mcand = fmaxf(m2[x], v + msafe);
        const float msafe_new = mcand == kNegInf ? 0.0f : mcand;
        const float alpha = __builtin_amdgcn_exp2f(m2[x] - msafe_new);
        lsum[x] *= alpha;
#pragma unroll
        for (int i2 = 0; i2 < ND; ++i2) o[x][i2] *= alpha;
        m2[x] = mcand;
        nms[x] = -msafe_new;
        const float shift = msafe - msafe_new;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) s4[x][t][r] += shift;
      }
    };
    if (!started) {  // wave-uniform: some row has not seen a visible key yet
      move_max();
      started = __ballot(m2[0] == kNegInf || m2[1] == kNegInf) == 0ull;
    }
    // p = 2^e packed as the P^T operands (k-slot e of lane group j4 is key 32 u + 4 j4 + e,
    // e < 4, or 32 u + 16 + 4 j4 + (e - 4)), and the lane's sum of the tile's p per row
    uint4 pb[NU][2];
    float ps[2];
    auto exps = [&]() {
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            pv[e] = __builtin_amdgcn_exp2f(s4[x][2 * u + (e >> 2)][e & 3]);
          // the first group's sum starts ps (0 + x is not folded: it would turn -0 into +0)
          const float s8 =
              ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
          ps[x] = u == 0 ? s8 : ps[x] + s8;
          pb[u][x] = make_uint4(Mfma<QT>::pack2(pv[0], pv[1]), Mfma<QT>::pack2(pv[2], pv[3]),
                                Mfma<QT>::pack2(pv[4], pv[5]), Mfma<QT>::pack2(pv[6], pv[7]));
        }
    };
    exps();
    if (__ballot(ps[0] > 256.0f || ps[1] > 256.0f) != 0ull) {
      move_max();
      exps();
    }
    lsum[0] += ps[0];
    lsum[1] += ps[1];
    // O^T += V^T P^T
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int i2 = 0; i2 < ND; ++i2) {
        o[0][i2] = Mfma<QT>::run(va[u][i2], pb[u][0], o[0][i2]);
        o[1][i2] = Mfma<QT>::run(va[u][i2], pb[u][1], o[1][i2]);
      }
    n_cur = n_nx;
    return n_cur > 0;
  };
  if (n_cur > 0)
    while (step(std::integral_constant<int, 0>{}) && step(std::integral_constant<int, 1>{})) {
    }

  // epilogue: reduce the lane-partial sums of each query over its 4 lane groups
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    float ls = lsum[x];
    ls += __shfl_xor(ls, 16, kWave);
    ls += __shfl_xor(ls, 32, kWave);
    if (q_ok[x]) {
      const int mq = m0 + 32 * ws + 16 * x + l16;
      const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
      QT* op = out.at(b, mq, h, 0);
#pragma unroll
      for (int i2 = 0; i2 < ND; ++i2) {
        uint2 w2;
        if constexpr (sizeof(QT) == 2) {
          if (gate.g != nullptr) {  // launch-uniform
            const float o4[4] = {o[x][i2][0] * inv, o[x][i2][1] * inv, o[x][i2][2] * inv,
                                 o[x][i2][3] * inv};
            *reinterpret_cast<uint2*>(op + 16 * i2 + 4 * j4) =
                gate_mix4(gate, b, mq, h, 16 * i2 + 4 * j4, o4);
            continue;
          }
        }
        w2.x = Mfma<QT>::pack2(o[x][i2][0] * inv, o[x][i2][1] * inv);
        w2.y = Mfma<QT>::pack2(o[x][i2][2] * inv, o[x][i2][3] * inv);
        *reinterpret_cast<uint2*>(op + 16 * i2 + 4 * j4) = w2;
      }
      if (lse != nullptr && j4 == 0)
        lse[(static_cast<int64_t>(b) * H + h) * M + mq] =
            ls > 0.0f ? (m2[x] + __builtin_log2f(ls)) * kLn2 : kNegInf;
    }
  }
}

// ---- fp32 MFMA kernel (fp32 q / k / v, head dim 64 or 128) ---------------------------------------
// One workgroup = one query group of up to 64 queries, 4 waves x 16 queries (the fp32 MFMA is
// 32 cycles long, so one operand read per MFMA costs little, and 16-query waves give config 1's
// 300 (group, head) items four times the waves).  K / V tiles of TK = 8 KiB / (4 D) keys go
// global -> LDS by buffer_load ... lds, double-buffered, every wave reading the same tile.
// S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x4_f32 with fp32 operands and fp32 P (P is
// not rounded, so the result stays within the fp32 bar).  The dims of a QK^T k-step are permuted
// (k-step 4 u + e takes dims 16 u + 4 j + e from lane group j), so a lane fetches the K
// operands of four k-steps with one 16-byte read; the keys of PV k-step (t, r) are 16 t + 4 j + r,
// so P^T is the lane's own S^T registers.
// LDS layout: copy instruction j (RPI rows of ROWB bytes) lands at j * PITCH, PITCH = 1024 +
// 16 RPI, so the PV operand rows 4 j + r of the 4 lane groups fall on 4 different bank ranges;
// K's 16-byte chunk c of row r is stored at chunk c ^ (r % 16) (through the copy's source
// offsets), which spreads the 16-row b128 reads.
constexpr int kF32Waves = 4;

template <int D>
struct F32Geom {
  static constexpr int ROWB = 4 * D;       // bytes per K / V row
  static constexpr int CPR = D / 4;        // 16-byte chunks per row
  static constexpr int TK = 8192 / ROWB;   // keys per tile (16 for D = 128, 32 for D = 64)
  static constexpr int RPI = 1024 / ROWB;  // rows per copy instruction
  static constexpr int PITCH = 1024 + 16 * RPI;
  static constexpr int NT = TK / 16;       // 16-key blocks per tile
  static constexpr int DU = D / 16;        // QK^T groups of 4 k-steps; PV d-tiles
  __device__ static int swz_k(int r) { return r & (CPR < 16 ? CPR - 1 : 15); }
  // byte offset of (row, 16-byte chunk slot) in a tile buffer
  __device__ static int at(int row, int slot) {
    return (row / RPI) * PITCH + (row % RPI) * ROWB + (slot << 4);
  }
};

// This wave's NI copy instructions of one fp32 tile: instruction j = NI w + jj lands at
// dst + j * PITCH (the M0 base steps by PITCH).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int PITCH>
__device__ __forceinline__ void dma_pitch2(const void* base, int rsb, int nrows, char* dst, int w,
                                           const int (&off)[2]) {
  const i32x4 r = buffer_desc(base, nrows * rsb);
  const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)) + PITCH * 2u * w)));
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
      "s_add_u32 m0, m0, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds"
      :
      : "s"(m0), "v"(off[0]), "v"(off[1]), "s"(r), "i"(PITCH)
      : "memory", "m0", "scc");
}
#pragma clang diagnostic pop

// Split fp32 calls: the B * H * MG items' T slots each, laid end to end (item-major, query group
// fastest, then head, then batch), are cut into `ranges` equal runs, one per workgroup, so that
// every CU gets the same number of selected blocks however few items the call has.  A workgroup
// walks the items its run touches; an item it covers whole is written out directly, a piece of
// an item is written as a record: per query row the unnormalised o (fp32, relative to m), the
// log2-domain reference m (-inf when the piece saw no key) and the sum l of its exponentials.  The
// first piece of run r goes to record 2 r, a later (its last) piece to record 2 r + 1, and
// sel_fwd_f32merge_kernel combines the records of every split item.
struct F32Split {
  float* rec;
  int64_t units;  // items * T
  int ranges;     // workgroups, <= units
};

template <int D>
constexpr int f32_rec_floats() {  // o [64][D], then (m, l) for 64 rows
  return 64 * D + 128;
}

// The item (b, query group g, head h) over its slots [lo, hi): writes out / lse when rec is
// null, else the piece's record at rec.
template <typename Acc, int D>
__device__ __forceinline__ void f32_piece(View4<const float> q, View4<float> out,
                                          float* __restrict__ lse, const Acc& acc, int M, int H,
                                          int G, int T, int chunk, float scale, int b, int g, int h,
                                          int lo, int hi, float* __restrict__ rec, char* lds) {
  using FG = F32Geom<D>;
  constexpr int CPR = FG::CPR, TK = FG::TK, RPI = FG::RPI, NT = FG::NT;
  constexpr int DU = FG::DU, PITCH = FG::PITCH;
  constexpr int NI = 8 / kF32Waves;  // copy instructions per wave per K or V tile
  static_assert(NI == 2, "two copy instructions per wave");
  constexpr int BUF = 8 * PITCH;  // lds: K buffers 0, 1; V buffers 2, 3
  const int tid = static_cast<int>(threadIdx.x), lane = lane_id(), w = tid / kWave;
  const int l16 = lane & 15, j4 = lane >> 4;
  const int m_end = min(g * G + G, M);
  const int qc = (g * G) / chunk;
  const int mq = g * G + 16 * w + l16;  // this lane's query (column l16 of the wave's block)
  const bool q_ok = 16 * w + l16 < G && mq < m_end;
  // Q^T operands: group u holds dims 16 u + 4 j4 + e, e < 4 (the k-steps 4 u + e)
  float4 qf[DU];
#pragma unroll
  for (int u = 0; u < DU; ++u)
    qf[u] = q_ok ? *reinterpret_cast<const float4*>(q.at(b, mq, h, 16 * u + 4 * j4))
                 : make_float4(0.f, 0.f, 0.f, 0.f);
  float c2 = scale * kLog2e;
  if (c2 < 0.0f) {  // the softmax works on s * c2 with c2 > 0: negate Q instead (exact)
    c2 = -c2;
#pragma unroll
    for (int u = 0; u < DU; ++u) qf[u] = make_float4(-qf[u].x, -qf[u].y, -qf[u].z, -qf[u].w);
  }
  // LDS read offsets (tile block t adds 16 rows: 16 / RPI instructions, a compile-time offset)
  int koff[DU];
#pragma unroll
  for (int u = 0; u < DU; ++u) koff[u] = FG::at(l16, (4 * u + j4) ^ FG::swz_k(l16));
  int voff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) voff[r] = FG::at(4 * j4 + r, 0) + 4 * l16;
  f32x4 o[DU];
#pragma unroll
  for (int i = 0; i < DU; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m2 = kNegInf, nms = 0.0f, thr = kNegInf, lsum = 0.0f;

  WaveWalk<Acc, TK> wk;
  wk.start_at(acc, b, g, h, lo, hi, qc);
  int n_cur = 0;
  int kdo[NI], vdo[NI];
  int rsk = 0, rsv = 0;
  if (wk.valid) {
    rsk = static_cast<int>(wk.br.sk) * 4;
    rsv = static_cast<int>(wk.br.sv) * 4;
#pragma unroll
    for (int jj = 0; jj < NI; ++jj) {
      const int row = (NI * w + jj) * RPI + lane / CPR, c = lane % CPR;
      kdo[jj] = row * rsk + ((c ^ FG::swz_k(row)) << 4);
      vdo[jj] = row * rsv + (c << 4);
    }
    dma_pitch2<PITCH>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(wk.tok0) * rsk,
                      rsk, wk.n, lds, w, kdo);
    dma_pitch2<PITCH>(static_cast<const char*>(wk.br.v) + static_cast<int64_t>(wk.tok0) * rsv,
                      rsv, wk.n, lds + 2 * BUF, w, vdo);
    n_cur = wk.n;
    wk.advance(acc, b, g, h, hi, qc);
  }
  __builtin_amdgcn_s_waitcnt(0);

  auto step = [&](auto BIc) -> bool {
    constexpr int BI = decltype(BIc)::value;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int n_nx = 0;
    if (wk.valid) {
      dma_pitch2<PITCH>(static_cast<const char*>(wk.br.k) + static_cast<int64_t>(wk.tok0) * rsk,
                        rsk, wk.n, lds + (BI ^ 1) * BUF, w, kdo);
      dma_pitch2<PITCH>(static_cast<const char*>(wk.br.v) + static_cast<int64_t>(wk.tok0) * rsv,
                        rsv, wk.n, lds + (2 + (BI ^ 1)) * BUF, w, vdo);
      n_nx = wk.n;
      wk.advance(acc, b, g, h, hi, qc);
    }
    const char* Kt = lds + BI * BUF;
    const char* Vt = lds + (2 + BI) * BUF;
    // S^T = K Q^T: lane holds keys 16 t + 4 j4 + r of query l16
    f32x4 s4[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      s4[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < DU; ++u) {
        const float4 a =
            *reinterpret_cast<const float4*>(Kt + koff[u] + t * (16 / RPI) * PITCH);
        s4[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, qf[u].x, s4[t], 0, 0, 0);
        s4[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, qf[u].y, s4[t], 0, 0, 0);
        s4[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, qf[u].z, s4[t], 0, 0, 0);
        s4[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, qf[u].w, s4[t], 0, 0, 0);
      }
    }
    if (n_cur < TK) {  // keys past n_cur are not visible (their rows read as 0)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (16 * t + 4 * j4 + r >= n_cur) s4[t][r] = kNegInf;
    }
    // online softmax in the log2 domain (the 16-bit kernels' scheme): e = s c2 - m, with m
    // raised only when some e exceeds 8
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_fmaf(s4[t][r], c2, nms);
        s4[t][r] = e;
        mx = fmaxf(mx, e);
      }
    if (__ballot(mx > thr) != 0ull) {
      const float msafe = m2 == kNegInf ? 0.0f : m2;
      float v = mx;
      v = fmaxf(v, __shfl_xor(v, 16, kWave));
      v = fmaxf(v, __shfl_xor(v, 32, kWave));
      const float mcand = fmaxf(m2, v + msafe);
      const float msafe_new = mcand == kNegInf ? 0.0f : mcand;
      const float alpha = __builtin_amdgcn_exp2f(m2 - msafe_new);
      lsum *= alpha;
#pragma unroll
      for (int i = 0; i < DU; ++i) o[i] *= alpha;
      m2 = mcand;
      nms = -msafe_new;
      thr = mcand == kNegInf ? kNegInf : 8.0f;
      const float shift = msafe - msafe_new;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) s4[t][r] += shift;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(s4[t][r]);
        s4[t][r] = p;
        lsum += p;
      }
    // O^T += V^T P^T: k-step (t, r) takes keys 16 t + 4 j + r, P^T from the lane's registers
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < DU; ++i) {
          const float a = *reinterpret_cast<const float*>(Vt + voff[r] + t * (16 / RPI) * PITCH +
                                                          64 * i);
          o[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, s4[t][r], o[i], 0, 0, 0);
        }
    n_cur = n_nx;
    return n_cur > 0;
  };
  if (n_cur > 0)
    while (step(std::integral_constant<int, 0>{}) && step(std::integral_constant<int, 1>{})) {
    }

  float ls = lsum;
  ls += __shfl_xor(ls, 16, kWave);
  ls += __shfl_xor(ls, 32, kWave);
  if (rec != nullptr) {  // a piece: every row of the record, unnormalised
    const int row = 16 * w + l16;
    float* ro = rec + row * D;
#pragma unroll
    for (int i = 0; i < DU; ++i)
      *reinterpret_cast<float4*>(ro + 16 * i + 4 * j4) =
          make_float4(o[i][0], o[i][1], o[i][2], o[i][3]);
    if (j4 == 0) *reinterpret_cast<float2*>(rec + 64 * D + 2 * row) = make_float2(m2, ls);
    return;
  }
  if (q_ok) {
    const float inv = ls > 0.0f ? 1.0f / ls : 0.0f;
    float* op = out.at(b, mq, h, 0);
#pragma unroll
    for (int i = 0; i < DU; ++i)
      *reinterpret_cast<float4*>(op + 16 * i + 4 * j4) =
          make_float4(o[i][0] * inv, o[i][1] * inv, o[i][2] * inv, o[i][3] * inv);
    if (lse != nullptr && j4 == 0)
      lse[(static_cast<int64_t>(b) * H + h) * M + mq] =
          ls > 0.0f ? (m2 + __builtin_log2f(ls)) * kLn2 : kNegInf;
  }
}

// One workgroup per (b, query group, head), launch order remapped so that an XCD's workgroups
// take consecutive groups of one head.
template <typename Acc, int D>
__global__ __launch_bounds__(kF32Waves * kWave, 2) void sel_fwd_f32mfma_kernel(
    View4<const float> q, View4<float> out, float* __restrict__ lse, Acc acc, int M, int H, int G,
    int MG, int T, int chunk, float scale) {
  __shared__ __align__(16) char lds[4 * 8 * F32Geom<D>::PITCH];
  int wi = xcd_remap(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int g = wi % MG; wi /= MG;
  const int h = wi % H;
  const int b = wi / H;
  f32_piece<Acc, D>(q, out, lse, acc, M, H, G, T, chunk, scale, b, g, h, 0, T, nullptr, lds);
}

// One workgroup per run of sp.units / sp.ranges slots (see F32Split); consecutive runs on one XCD.
template <typename Acc, int D>
__global__ __launch_bounds__(kF32Waves * kWave, 2) void sel_fwd_f32split_kernel(
    View4<const float> q, View4<float> out, float* __restrict__ lse, Acc acc, int M, int H, int G,
    int MG, int T, int chunk, float scale, F32Split sp) {
  __shared__ __align__(16) char lds[4 * 8 * F32Geom<D>::PITCH];
  const int r = xcd_remap(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int64_t u0 = static_cast<int64_t>(r) * sp.units / sp.ranges;
  const int64_t u1 = static_cast<int64_t>(r + 1) * sp.units / sp.ranges;
  bool first = true;
  for (int64_t i = u0 / T; i * T < u1; ++i) {
    const int lo = static_cast<int>(u0 > i * T ? u0 - i * T : 0);
    const int hi = static_cast<int>(u1 - i * T < T ? u1 - i * T : T);
    float* rec = nullptr;
    if (lo > 0 || hi < T)
      rec = sp.rec + (2 * static_cast<int64_t>(r) + (first ? 0 : 1)) * f32_rec_floats<D>();
    if (!first) __syncthreads();  // the previous piece's last tile reads are done everywhere
    const int g = static_cast<int>(i % MG);
    const int h = static_cast<int>((i / MG) % H);
    const int b = static_cast<int>(i / (static_cast<int64_t>(MG) * H));
    f32_piece<Acc, D>(q, out, lse, acc, M, H, G, T, chunk, scale, b, g, h, lo, hi, rec, lds);
    first = false;
  }
}

// The split items (those whose slots span two or more runs): out = sum_r 2^(m_r - m) o_r /
// sum_r 2^(m_r - m) l_r over the records r of the item, m = the largest m_r with l_r > 0, and
// lse = (m + log2 of that sum) ln 2 (0 and -inf when no piece saw a key).  One thread per 4 dims
// of a query row; workgroup x covers rows RPW (x % (64 / RPW)) .. of item x / (64 / RPW).
template <int D>
__global__ __launch_bounds__(256) void sel_fwd_f32merge_kernel(View4<float> out,
                                                               float* __restrict__ lse, int M,
                                                               int H, int G, int MG, int T,
                                                               F32Split sp) {
  constexpr int REC = f32_rec_floats<D>(), TPR = D / 4, RPW = 256 / TPR, WPI = 64 / RPW;
  const int64_t i = blockIdx.x / WPI;
  const int64_t s0 = i * T;
  auto run_of = [&](int64_t s) {  // r with floor(r U / R) <= s < floor((r + 1) U / R)
    return ((s + 1) * sp.ranges + sp.units - 1) / sp.units - 1;
  };
  const int64_t ra = run_of(s0), rb = run_of(s0 + T - 1);
  if (ra == rb) return;  // written whole by its run
  const bool ra_first = ra * sp.units / sp.ranges == s0;
  const int tid = static_cast<int>(threadIdx.x);
  const int row = static_cast<int>(blockIdx.x % WPI) * RPW + tid / TPR, c4 = tid % TPR;
  const int g = static_cast<int>(i % MG);
  const int h = static_cast<int>((i / MG) % H);
  const int b = static_cast<int>(i / (static_cast<int64_t>(MG) * H));
  const int mq = g * G + row;
  if (row >= G || mq >= M) return;
  const float* rp = sp.rec + (2 * ra + (ra_first ? 0 : 1)) * REC;
  float mx = kNegInf, l = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t r = ra; r <= rb; ++r, rp = sp.rec + 2 * r * REC) {
    const float2 ml = *reinterpret_cast<const float2*>(rp + 64 * D + 2 * row);
    const float4 x = *reinterpret_cast<const float4*>(rp + row * D + 4 * c4);
    if (!(ml.y > 0.0f)) continue;
    if (ml.x > mx) {  // a new reference: rescale what is summed so far
      const float f = __builtin_amdgcn_exp2f(mx - ml.x);
      l *= f;
      acc.x *= f; acc.y *= f; acc.z *= f; acc.w *= f;
      mx = ml.x;
    }
    const float wgt = __builtin_amdgcn_exp2f(ml.x - mx);
    l += wgt * ml.y;
    acc.x += wgt * x.x; acc.y += wgt * x.y; acc.z += wgt * x.z; acc.w += wgt * x.w;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  *reinterpret_cast<float4*>(out.at(b, mq, h, 4 * c4)) =
      make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  if (lse != nullptr && c4 == 0)
    lse[(static_cast<int64_t>(b) * H + h) * M + mq] =
        l > 0.0f ? (mx + __builtin_log2f(l)) * kLn2 : kNegInf;
}

// ---- VALU kernel (fp32 arithmetic, any head dim <= 256, any strides) -------------------------
constexpr int kValuKeys = 32;

template <typename QT, typename Acc, int DQ>
__global__ __launch_bounds__(256) void sel_fwd_valu_kernel(View4<const QT> q, View4<QT> out,
                                                           float* __restrict__ lse, Acc acc, int M,
                                                           int H, int D, int G, int MG, int T,
                                                           int chunk, float scale, int nsub,
                                                           int64_t kv_sd) {
  constexpr int DP = 4 * DQ;
  __shared__ float Ks[kValuKeys * DP];
  __shared__ float Vs[kValuKeys * DP];
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
  if (sub == 0) acc.touch(b, g, h, T);
  const int qi = tid >> 2, part = tid & 3;
  const int my_q = m0 + qi;
  const bool q_ok = my_q < m_end;
  const int d0 = part * DQ;

  float qr[DQ], o[DQ];
#pragma unroll
  for (int i = 0; i < DQ; ++i) {
    const int d = d0 + i;
    qr[i] = (q_ok && d < D) ? to_f32<QT>(*q.at(b, my_q, h, d)) : 0.0f;
    o[i] = 0.0f;
  }
  float m = kNegInf, l = 0.0f;
  for (TileIt it = first_tile(acc, b, g, h, T, qc, 0); it.valid;) {
    // process the tile in sub-tiles of kValuKeys tokens
    for (int k0 = 0; k0 < it.n; k0 += kValuKeys) {
      const int nk = min(kValuKeys, it.n - k0);
      __syncthreads();
      for (int i = tid; i < kValuKeys * DP; i += 256) {
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
      float s[kValuKeys];
#pragma unroll
      for (int kk = 0; kk < kValuKeys; ++kk) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < DQ; ++i) a = __builtin_fmaf(qr[i], Ks[kk * DP + d0 + i], a);
        a += __shfl_xor(a, 1, kWave);
        a += __shfl_xor(a, 2, kWave);
        s[kk] = kk < nk ? a * scale : kNegInf;
      }
      float mt = kNegInf;
#pragma unroll
      for (int kk = 0; kk < kValuKeys; ++kk) mt = fmaxf(mt, s[kk]);
      const float mnew = fmaxf(m, mt);
      const float alpha = (m == kNegInf) ? 0.0f : expf(m - mnew);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < DQ; ++i) o[i] *= alpha;
#pragma unroll
      for (int kk = 0; kk < kValuKeys; ++kk) {
        const float p = (s[kk] == kNegInf) ? 0.0f : expf(s[kk] - mnew);
        l += p;
#pragma unroll
        for (int i = 0; i < DQ; ++i) o[i] = __builtin_fmaf(p, Vs[kk * DP + d0 + i], o[i]);
      }
      m = mnew;
    }
    it = next_tile(acc, it, b, g, h, T, qc);
  }
  if (q_ok) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      const int d = d0 + i;
      if (d < D) *out.at(b, my_q, h, d) = from_f32<QT>(o[i] * inv);
    }
    if (lse != nullptr && part == 0)
      lse[(static_cast<int64_t>(b) * H + h) * M + my_q] = l > 0.0f ? m + logf(l) : kNegInf;
  }
}

// ---- launch helpers -------------------------------------------------------------------------
struct Geom {
  int B, M, H, D, G, MG, T, nsub;
  int64_t items;
};

inline int geom(const omm_view4& q, int64_t MGv, int64_t T, int G, Geom& g) {
  g.B = static_cast<int>(q.size[0]);
  g.M = static_cast<int>(q.size[1]);
  g.H = static_cast<int>(q.size[2]);
  g.D = static_cast<int>(q.size[3]);
  g.G = G;
  g.MG = static_cast<int>(MGv);
  g.T = static_cast<int>(T);
  g.nsub = (G + 63) / 64;
  g.items = static_cast<int64_t>(g.B) * g.H * g.MG * g.nsub;
  OMM_REQUIRE(g.items <= 2147483647ll, OMM_EUNSUPPORTED, "selection: grid too large");
  return OMM_OK;
}

// out = g0 * o_cmp + g1 * out + g2 * o_swa in place, fp32 arithmetic and one rounding: the gated
// mix after the register-staged kernels, which keep no gate code.  Their epilogue would read
// o_cmp / o_swa at the end of every workgroup; on the fp8 AR call that cost ~37 us against
// ~8 us for this pass (and the gate code slowed the ungated kernel too).  One thread per 8 dims
// of one (b, m, h).
__global__ __launch_bounds__(256) void branch_mix_kernel(GateArgs ga, View4<bf16_t> out, int M,
                                                         int H, int C8, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int c = static_cast<int>(i % C8);
    int64_t r = i / C8;
    const int h = static_cast<int>(r % H);
    r /= H;
    const int m = static_cast<int>(r % M);
    const int b = static_cast<int>(r / M);
    const uint16_t* gp =
        reinterpret_cast<const uint16_t*>(ga.g + b * ga.gs0 + m * ga.gs1 + h * ga.gs2);
    const float g0 = bf16_bits_to_f32(gp[0]), g1 = bf16_bits_to_f32(gp[ga.gs3]);
    const float g2 = bf16_bits_to_f32(gp[2 * ga.gs3]);
    uint4* op = reinterpret_cast<uint4*>(out.at(b, m, h, 8 * c));
    const uint4 sv = *op;
    const uint4 cv = *reinterpret_cast<const uint4*>(ga.oc + b * ga.cs0 + m * ga.cs1 + h * ga.cs2 + 8 * c);
    const uint4 wv = *reinterpret_cast<const uint4*>(ga.ow + b * ga.ws0 + m * ga.ws1 + h * ga.ws2 + 8 * c);
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w}, cw[4] = {cv.x, cv.y, cv.z, cv.w};
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t res[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float r2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float cf = __builtin_bit_cast(float, e ? cw[k] & 0xffff0000u : cw[k] << 16);
        const float sf = __builtin_bit_cast(float, e ? sw[k] & 0xffff0000u : sw[k] << 16);
        const float wf = __builtin_bit_cast(float, e ? ww[k] & 0xffff0000u : ww[k] << 16);
        r2[e] = __builtin_fmaf(g2, wf, __builtin_fmaf(g1, sf, g0 * cf));
      }
      res[k] = pack_bf16x2(r2[0], r2[1]);
    }
    *op = make_uint4(res[0], res[1], res[2], res[3]);
  }
}

int launch_mix(const omm_view4& out, const GateArgs& gate, hipStream_t s) {
  const int B = static_cast<int>(out.size[0]), M = static_cast<int>(out.size[1]);
  const int H = static_cast<int>(out.size[2]), C8 = static_cast<int>(out.size[3] / 8);
  const int64_t n = static_cast<int64_t>(B) * M * H * C8;
  const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv64(n, 256), 4096));
  branch_mix_kernel<<<blocks, 256, 0, s>>>(gate, make_view<bf16_t>(out), M, H, C8, n);
  return check_launch("selection attention (branch mix)");
}

template <typename QT, typename Acc, int D>
int launch_mfma(const Geom& gm, const omm_view4& q, const omm_view4& out, float* lse,
                const Acc& acc, int chunk, float scale, hipStream_t s, const GateArgs& gate) {
  sel_fwd_mfma_kernel<QT, Acc, D><<<static_cast<unsigned>(gm.items), kMfmaThreads, 0, s>>>(
      make_view<const QT>(q), make_view<QT>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG, gm.T, chunk,
      scale, gm.nsub);
  const int rc = check_launch("selection attention (mfma)");
  if constexpr (sizeof(QT) == 2)
    if (rc == OMM_OK && gate.g != nullptr) return launch_mix(out, gate, s);
  return rc;
}

// fp8 pages with the fp8 QK^T (queries quantised per row), head dim 64 or 128
template <typename Acc, int D>
int launch_qk8(const Geom& gm, const omm_view4& q, const omm_view4& out, float* lse,
               const Acc& acc, int chunk, float scale, hipStream_t s, const GateArgs& gate) {
  sel_fwd_mfma_kernel<bf16_t, Acc, D, true><<<static_cast<unsigned>(gm.items), kMfmaThreads, 0, s>>>(
      make_view<const bf16_t>(q), make_view<bf16_t>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG, gm.T,
      chunk, scale, gm.nsub);
  const int rc = check_launch("selection attention (fp8 QK)");
  if (rc == OMM_OK && gate.g != nullptr) return launch_mix(out, gate, s);
  return rc;
}

template <typename QT, typename Acc, int D>
int launch_dma(const Geom& gm, const omm_view4& q, const omm_view4& out, float* lse,
               const Acc& acc, int chunk, float scale, hipStream_t s, const GateArgs& gate) {
  if (gm.nsub >= 2) {  // two 64-query subgroups per workgroup
    const int64_t grid = gm.items / gm.nsub * ((gm.nsub + 1) / 2);
    sel_fwd_dma_kernel<QT, Acc, D, 4><<<static_cast<unsigned>(grid), 4 * kWave, 0, s>>>(
        make_view<const QT>(q), make_view<QT>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG, gm.T,
        chunk, scale, gm.nsub, gate);
  } else {
    sel_fwd_dma_kernel<QT, Acc, D, 2><<<static_cast<unsigned>(gm.items), 2 * kWave, 0, s>>>(
        make_view<const QT>(q), make_view<QT>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG, gm.T,
        chunk, scale, gm.nsub, gate);
  }
  return check_launch("selection attention (dma)");
}

// Compute units of the current device (0 when the runtime cannot say), cached per device.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// A split fp32 call runs kF32RunsPerCu equal runs per CU when it has fewer than kF32SplitBelow
// items per CU (one item per workgroup leaves CUs idle or doubly loaded there: config 1's 300
// items take as long as 500 on 256 CUs).  0: no split.
constexpr int kF32RunsPerCu = 2;
constexpr int kF32SplitBelow = 4;

inline int f32_split_runs(int64_t items, int64_t T) {
  const int cus = device_cus();
  if (cus <= 0 || items <= 0 || T <= 0 || items >= int64_t{kF32SplitBelow} * cus) return 0;
  const int64_t units = items * T;
  const int64_t runs = int64_t{kF32RunsPerCu} * cus;
  return static_cast<int>(runs < units ? runs : units);
}

inline size_t f32_split_bytes(int runs, int64_t D) {
  return static_cast<size_t>(2) * runs * static_cast<size_t>(64 * D + 128) * sizeof(float);
}

template <typename Acc>
int launch_f32mfma(const Geom& gm, const omm_view4& q, const omm_view4& out, float* lse,
                   const Acc& acc, int chunk, float scale, hipStream_t s, const F32Split* sp) {
  if (sp != nullptr) {
    const unsigned runs = static_cast<unsigned>(sp->ranges);
    const unsigned items = static_cast<unsigned>(gm.items);
    if (gm.D == 128) {
      sel_fwd_f32split_kernel<Acc, 128><<<runs, kF32Waves * kWave, 0, s>>>(
          make_view<const float>(q), make_view<float>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG,
          gm.T, chunk, scale, *sp);
      sel_fwd_f32merge_kernel<128><<<items * 8, 256, 0, s>>>(make_view<float>(out), lse, gm.M,
                                                            gm.H, gm.G, gm.MG, gm.T, *sp);
    } else {
      sel_fwd_f32split_kernel<Acc, 64><<<runs, kF32Waves * kWave, 0, s>>>(
          make_view<const float>(q), make_view<float>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG,
          gm.T, chunk, scale, *sp);
      sel_fwd_f32merge_kernel<64><<<items * 4, 256, 0, s>>>(make_view<float>(out), lse, gm.M,
                                                           gm.H, gm.G, gm.MG, gm.T, *sp);
    }
    return check_launch("selection attention (fp32 mfma, split)");
  }
  const unsigned grid = static_cast<unsigned>(gm.items);
  if (gm.D == 128)
    sel_fwd_f32mfma_kernel<Acc, 128><<<grid, kF32Waves * kWave, 0, s>>>(
        make_view<const float>(q), make_view<float>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG, gm.T,
        chunk, scale);
  else
    sel_fwd_f32mfma_kernel<Acc, 64><<<grid, kF32Waves * kWave, 0, s>>>(
        make_view<const float>(q), make_view<float>(out), lse, acc, gm.M, gm.H, gm.G, gm.MG, gm.T,
        chunk, scale);
  return check_launch("selection attention (fp32 mfma)");
}

template <typename QT, typename Acc>
int launch_valu(const Geom& gm, const omm_view4& q, const omm_view4& out, float* lse,
                const Acc& acc, int chunk, float scale, int64_t kv_sd, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(gm.items);
  if (gm.D <= 64) {
    sel_fwd_valu_kernel<QT, Acc, 16><<<grid, 256, 0, s>>>(make_view<const QT>(q), make_view<QT>(out),
                                                          lse, acc, gm.M, gm.H, gm.D, gm.G, gm.MG,
                                                          gm.T, chunk, scale, gm.nsub, kv_sd);
  } else if (gm.D <= 128) {
    sel_fwd_valu_kernel<QT, Acc, 32><<<grid, 256, 0, s>>>(make_view<const QT>(q), make_view<QT>(out),
                                                          lse, acc, gm.M, gm.H, gm.D, gm.G, gm.MG,
                                                          gm.T, chunk, scale, gm.nsub, kv_sd);
  } else {
    sel_fwd_valu_kernel<QT, Acc, 64><<<grid, 256, 0, s>>>(make_view<const QT>(q), make_view<QT>(out),
                                                          lse, acc, gm.M, gm.H, gm.D, gm.G, gm.MG,
                                                          gm.T, chunk, scale, gm.nsub, kv_sd);
  }
  return check_launch("selection attention (valu)");
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// MFMA path preconditions on q / out (16-byte rows, unit dim stride).
inline bool qo_mfma_ok(const omm_view4& q, const omm_view4& out) {
  return q.stride[3] == 1 && out.stride[3] == 1 && aligned16(q.data) && aligned16(out.data) &&
         q.stride[0] % 8 == 0 && q.stride[1] % 8 == 0 && q.stride[2] % 8 == 0 &&
         out.stride[0] % 4 == 0 && out.stride[1] % 4 == 0 && out.stride[2] % 4 == 0;
}

// kv_row_bytes: the larger K / V row stride in bytes (the DMA kernel's 32-bit tile offsets and
// its zero-fill bound need TK rows to fit in 2^31 bytes and rows no shorter than D elements).
template <typename QT, typename Acc>
int dispatch(const Geom& gm, const omm_view4& q, const omm_view4& out, float* lse, const Acc& acc,
             int chunk, float scale, bool mfma_ok, int64_t kv_sd, int64_t kv_row_bytes,
             hipStream_t s, const GateArgs& gate = GateArgs{}) {
  if constexpr (sizeof(QT) == 2) {
    // the MFMA softmax needs a finite non-zero scale (its masking uses -inf scores)
    const bool ok = mfma_ok && scale != 0.0f && __builtin_isfinite(scale);
    if constexpr (sizeof(typename Acc::KV) == 2) {
      const bool rows_ok = kv_row_bytes >= 2 * gm.D && kv_row_bytes * 64 < (int64_t{1} << 31);
      if (ok && rows_ok && gm.D == 128)
        return launch_dma<QT, Acc, 128>(gm, q, out, lse, acc, chunk, scale, s, gate);
      if (ok && rows_ok && gm.D == 64)
        return launch_dma<QT, Acc, 64>(gm, q, out, lse, acc, chunk, scale, s, gate);
    }
    if (ok && gm.D == 128) return launch_mfma<QT, Acc, 128>(gm, q, out, lse, acc, chunk, scale, s, gate);
    if (ok && gm.D == 64) return launch_mfma<QT, Acc, 64>(gm, q, out, lse, acc, chunk, scale, s, gate);
  }
  OMM_REQUIRE(gate.g == nullptr, OMM_EUNSUPPORTED,
              "selection attention: the gated epilogue needs the MFMA path (bf16 q / out with "
              "16-byte rows, head dim 64 or 128, a finite non-zero scale)");
  return launch_valu<QT, Acc>(gm, q, out, lse, acc, chunk, scale, kv_sd, s);
}

int check_q_out(const char* op, const omm_view4* q, const omm_view4* out) {
  OMM_REQUIRE(q != nullptr && out != nullptr, OMM_EINVAL, "%s: null q/out", op);
  for (int i = 0; i < 4; ++i)
    OMM_REQUIRE(q->size[i] == out->size[i], OMM_EINVAL, "%s: out must have q's shape", op);
  OMM_REQUIRE(q->size[3] >= 1 && q->size[3] <= 256, OMM_EUNSUPPORTED,
              "%s: head dim must be in [1, 256], got %lld", op, (long long)q->size[3]);
  return OMM_OK;
}

template <typename QT>
int sel_fwd_typed(const omm_view4& q, const omm_view4& k, const omm_view4& v, const omm_view4& ids,
                  int bs, int chunk, bool causal, int G, float scale, const omm_view4& out,
                  float* lse, hipStream_t s, const GateArgs& gate = GateArgs{},
                  void* ws = nullptr, size_t ws_bytes = 0) {
  Geom gm;
  int rc = geom(q, ids.size[1], ids.size[3], G, gm);
  if (rc) return rc;
  OMM_REQUIRE(ids_offsets_fit32(ids), OMM_EUNSUPPORTED,
              "selection attention: block_indices must span fewer than 2^31 elements");
  OMM_REQUIRE(kv_offsets_fit32(k, v), OMM_EUNSUPPORTED,
              "selection attention: a (batch, head) slice of k / v must span fewer than 2^32 "
              "elements");
  DenseAcc<QT> acc{make_view<const QT>(k), make_view<const QT>(v),
                   static_cast<const int32_t*>(ids.data), ids.stride[0], ids.stride[1],
                   ids.stride[2], ids.stride[3], static_cast<int>(k.size[1]), bs,
                   causal ? chunk : 1, causal};
  const bool kv_ok = k.stride[3] == 1 && v.stride[3] == 1 && aligned16(k.data) &&
                     aligned16(v.data) && k.stride[0] % 8 == 0 && k.stride[1] % 8 == 0 &&
                     k.stride[2] % 8 == 0 && v.stride[0] % 8 == 0 && v.stride[1] % 8 == 0 &&
                     v.stride[2] % 8 == 0;
  const bool mfma = sizeof(QT) == 2 && kv_ok && qo_mfma_ok(q, out);
  if constexpr (sizeof(QT) == 4) {
    // fp32 on MFMA: 16-byte rows of unit dim stride, groups of at most 64 queries, head dim 64 or
    // 128, a finite non-zero scale (the masking uses -inf scores), 32-bit tile offsets
    auto rows16 = [](const omm_view4& x) {
      return x.stride[3] == 1 && aligned16(x.data) && x.stride[0] % 4 == 0 &&
             x.stride[1] % 4 == 0 && x.stride[2] % 4 == 0;
    };
    const int64_t rb = 4 * (k.stride[1] > v.stride[1] ? k.stride[1] : v.stride[1]);
    if (rows16(q) && rows16(out) && rows16(k) && rows16(v) && G <= 64 &&
        (gm.D == 64 || gm.D == 128) && scale != 0.0f && __builtin_isfinite(scale) &&
        rb >= 4 * gm.D && rb * 32 < (int64_t{1} << 31)) {
      // the split needs the caller's workspace (omm_sel_fwd_workspace_bytes) and one item per
      // 64-query group
      const int runs = ws != nullptr && gm.nsub == 1 ? f32_split_runs(gm.items, gm.T) : 0;
      if (runs > 0 && ws_bytes >= f32_split_bytes(runs, gm.D)) {
        const F32Split sp{static_cast<float*>(ws), gm.items * gm.T, runs};
        return launch_f32mfma(gm, q, out, lse, acc, causal ? chunk : 1, scale, s, &sp);
      }
      return launch_f32mfma(gm, q, out, lse, acc, causal ? chunk : 1, scale, s, nullptr);
    }
  }
  // the VALU kernel reads K and V with K's dim stride
  OMM_REQUIRE(mfma || k.stride[3] == v.stride[3], OMM_EUNSUPPORTED,
              "selection attention: k and v need the same dim stride");
  const int64_t row_bytes = 2 * (k.stride[1] > v.stride[1] ? k.stride[1] : v.stride[1]);
  return dispatch<QT>(gm, q, out, lse, acc, causal ? chunk : 1, scale, mfma, k.stride[3],
                      row_bytes, s, gate);
}

// The gate views of a gated call against q and out: gates [B, M, H, 3] bf16, o_cmp / o_swa of q's
// shape with unit dim stride and 16-byte rows; out may not overlap o_cmp or o_swa unless it is
// the very same view and `same_ok` (an epilogue that reads each element before writing it).
int gate_args(const char* op, const omm_view4* q, const omm_view4* gates, const omm_view4* o_cmp,
              const omm_view4* o_swa, const omm_view4* out, bool same_ok, GateArgs& ga) {
  OMM_REQUIRE(q != nullptr && out != nullptr && gates != nullptr && o_cmp != nullptr &&
                  o_swa != nullptr, OMM_EINVAL, "%s: null argument", op);
  OMM_REQUIRE(gates->size[0] == q->size[0] && gates->size[1] == q->size[1] &&
                  gates->size[2] == q->size[2] && gates->size[3] == 3,
              OMM_EINVAL, "%s: gates must be [B, M, H, 3]", op);
  for (const omm_view4* o : {o_cmp, o_swa}) {
    for (int i = 0; i < 4; ++i)
      OMM_REQUIRE(o->size[i] == q->size[i], OMM_EINVAL, "%s: o_cmp / o_swa must have q's shape", op);
    OMM_REQUIRE(o->stride[3] == 1 && o->stride[0] % 8 == 0 && o->stride[1] % 8 == 0 &&
                    o->stride[2] % 8 == 0 && (reinterpret_cast<uintptr_t>(o->data) & 15u) == 0,
                OMM_EUNSUPPORTED,
                "%s: o_cmp / o_swa need unit dim stride and 16-byte aligned rows", op);
    const bool same = o->data == out->data && o->stride[0] == out->stride[0] &&
                      o->stride[1] == out->stride[1] && o->stride[2] == out->stride[2] &&
                      o->stride[3] == out->stride[3];
    if (views_overlap(*o, *out, 2))
      OMM_REQUIRE(same && same_ok, OMM_EINVAL, "%s: out overlaps o_cmp or o_swa", op);
  }
  ga.g = static_cast<const bf16_t*>(gates->data);
  ga.gs0 = gates->stride[0]; ga.gs1 = gates->stride[1]; ga.gs2 = gates->stride[2];
  ga.gs3 = gates->stride[3];
  ga.oc = static_cast<const bf16_t*>(o_cmp->data);
  ga.cs0 = o_cmp->stride[0]; ga.cs1 = o_cmp->stride[1]; ga.cs2 = o_cmp->stride[2];
  ga.ow = static_cast<const bf16_t*>(o_swa->data);
  ga.ws0 = o_swa->stride[0]; ga.ws1 = o_swa->stride[1]; ga.ws2 = o_swa->stride[2];
  return OMM_OK;
}

}  // namespace
}  // namespace omm

extern "C" size_t omm_sel_fwd_workspace_bytes(int64_t B, int64_t M, int64_t H, int64_t D,
                                               int64_t T, int32_t dtype, int32_t group_size) {
  using namespace omm;
  if (dtype != OMM_F32 || (D != 64 && D != 128) || group_size < 1 || group_size > 64 || B <= 0 ||
      M <= 0 || H <= 0 || T <= 0)
    return 0;
  const int runs = f32_split_runs(B * H * cdiv64(M, group_size), T);
  return runs > 0 ? f32_split_bytes(runs, D) : 0;
}

extern "C" int omm_sel_fwd(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                           const omm_view4* ids, int32_t dtype, int32_t block_size,
                           int32_t chunk_size, int32_t causal, int32_t group_size, float scale,
                           const omm_view4* out, float* lse, void* stream) {
  return omm_sel_fwd_ws(q, k, v, ids, dtype, block_size, chunk_size, causal, group_size, scale,
                        out, lse, nullptr, 0, stream);
}

extern "C" int omm_sel_fwd_ws(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                              const omm_view4* ids, int32_t dtype, int32_t block_size,
                              int32_t chunk_size, int32_t causal, int32_t group_size, float scale,
                              const omm_view4* out, float* lse, void* workspace,
                              size_t workspace_bytes, void* stream) {
  using namespace omm;
  OMM_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, OMM_EINVAL,
              "omm_sel_fwd: workspace must be 16-byte aligned");
  int rc = check_q_out("omm_sel_fwd", q, out);
  if (rc) return rc;
  OMM_REQUIRE(k != nullptr && v != nullptr && ids != nullptr, OMM_EINVAL, "omm_sel_fwd: null view");
  const int64_t B = q->size[0], M = q->size[1], H = q->size[2], D = q->size[3];
  for (int i = 0; i < 4; ++i)
    OMM_REQUIRE(k->size[i] == v->size[i], OMM_EINVAL, "omm_sel_fwd: k and v must have the same shape");
  OMM_REQUIRE(k->size[0] == B && k->size[2] == H && k->size[3] == D, OMM_EINVAL,
              "omm_sel_fwd: expected k/v [B,N,H,D] compatible with q");
  OMM_REQUIRE(group_size >= 1 && block_size >= 1 && chunk_size >= 1, OMM_EINVAL,
              "omm_sel_fwd: group_size, block_size and chunk_size must be >= 1");
  const int64_t MG = cdiv64(M, group_size);
  OMM_REQUIRE(ids->size[0] == B && ids->size[1] == MG && ids->size[2] == H && ids->size[3] >= 1,
              OMM_EINVAL, "omm_sel_fwd: block_indices must be [%lld,%lld,%lld,T>=1]", (long long)B,
              (long long)MG, (long long)H);
  OMM_REQUIRE(k->size[1] <= 2147483647ll && M <= 2147483647ll, OMM_EUNSUPPORTED, "omm_sel_fwd: too long");
  if (B == 0 || M == 0 || H == 0) return OMM_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case OMM_BF16:
      return sel_fwd_typed<bf16_t>(*q, *k, *v, *ids, block_size, chunk_size, causal != 0, group_size,
                                   scale, *out, lse, s);
    case OMM_F16:
      return sel_fwd_typed<f16_t>(*q, *k, *v, *ids, block_size, chunk_size, causal != 0, group_size,
                                  scale, *out, lse, s);
    case OMM_F32:
      return sel_fwd_typed<float>(*q, *k, *v, *ids, block_size, chunk_size, causal != 0, group_size,
                                  scale, *out, lse, s, GateArgs{}, workspace, workspace_bytes);
    default: return set_error(OMM_EINVAL, "omm_sel_fwd: unsupported dtype %d", dtype);
  }
}

extern "C" int omm_sel_fwd_gated(const omm_view4* q, const omm_view4* k, const omm_view4* v,
                                 const omm_view4* ids, int32_t block_size, int32_t chunk_size,
                                 int32_t causal, int32_t group_size, float scale,
                                 const omm_view4* gates, const omm_view4* o_cmp,
                                 const omm_view4* o_swa, const omm_view4* out, float* lse,
                                 void* stream) {
  using namespace omm;
  int rc = check_q_out("omm_sel_fwd_gated", q, out);
  if (rc) return rc;
  GateArgs ga;
  // the register-staged fallback mixes in a second pass after writing out: no overlap at all
  rc = gate_args("omm_sel_fwd_gated", q, gates, o_cmp, o_swa, out, false, ga);
  if (rc) return rc;
  OMM_REQUIRE(k != nullptr && v != nullptr && ids != nullptr, OMM_EINVAL,
              "omm_sel_fwd_gated: null view");
  const int64_t B = q->size[0], M = q->size[1], H = q->size[2], D = q->size[3];
  for (int i = 0; i < 4; ++i)
    OMM_REQUIRE(k->size[i] == v->size[i], OMM_EINVAL,
                "omm_sel_fwd_gated: k and v must have the same shape");
  OMM_REQUIRE(k->size[0] == B && k->size[2] == H && k->size[3] == D, OMM_EINVAL,
              "omm_sel_fwd_gated: expected k/v [B,N,H,D] compatible with q");
  OMM_REQUIRE(group_size >= 1 && block_size >= 1 && chunk_size >= 1, OMM_EINVAL,
              "omm_sel_fwd_gated: group_size, block_size and chunk_size must be >= 1");
  const int64_t MG = cdiv64(M, group_size);
  OMM_REQUIRE(ids->size[0] == B && ids->size[1] == MG && ids->size[2] == H && ids->size[3] >= 1,
              OMM_EINVAL, "omm_sel_fwd_gated: block_indices must be [%lld,%lld,%lld,T>=1]",
              (long long)B, (long long)MG, (long long)H);
  OMM_REQUIRE(k->size[1] <= 2147483647ll && M <= 2147483647ll, OMM_EUNSUPPORTED,
              "omm_sel_fwd_gated: too long");
  if (B == 0 || M == 0 || H == 0) return OMM_OK;
  return sel_fwd_typed<bf16_t>(*q, *k, *v, *ids, block_size, chunk_size, causal != 0, group_size,
                               scale, *out, lse, static_cast<hipStream_t>(stream), ga);
}

extern "C" int omm_sel_fwd_ptr(const omm_view4* q, const int64_t* ptr_k, const int64_t* ptr_v,
                               const int64_t* ptr_stride, int64_t T, int32_t block_size,
                               int32_t group_size, int64_t stride_bn, int64_t stride_bd,
                               float scale, const omm_view4* out, float* lse, void* stream) {
  using namespace omm;
  int rc = check_q_out("omm_sel_fwd_ptr", q, out);
  if (rc) return rc;
  OMM_REQUIRE(ptr_k != nullptr && ptr_v != nullptr && ptr_stride != nullptr, OMM_EINVAL,
              "omm_sel_fwd_ptr: null pointer table");
  OMM_REQUIRE(group_size >= 1 && block_size >= 1 && T >= 1, OMM_EINVAL,
              "omm_sel_fwd_ptr: group_size, block_size and T must be >= 1");
  OMM_REQUIRE(stride_bn >= 0 && stride_bd >= 0, OMM_EINVAL, "omm_sel_fwd_ptr: negative stride");
  Geom gm;
  rc = geom(*q, cdiv64(q->size[1], group_size), T, group_size, gm);
  if (rc) return rc;
  if (gm.items == 0) return OMM_OK;
  PtrAcc acc{ptr_k, ptr_v, ptr_stride[0], ptr_stride[1], ptr_stride[2], ptr_stride[3], stride_bn,
             block_size};
  // the MFMA kernels need 16-byte row strides; a block address that is not 16-byte aligned
  // (any bf16 address is accepted) is detected per block on the device and copied with 2-byte
  // loads
  const bool mfma = stride_bd == 1 && stride_bn % 8 == 0 && qo_mfma_ok(*q, *out);
  return dispatch<bf16_t>(gm, *q, *out, lse, acc, 1, scale, mfma, stride_bd, 2 * stride_bn,
                          static_cast<hipStream_t>(stream));
}

namespace omm {
namespace {
int sel_fwd_paged_impl(const omm_view4* q, const omm_view4* ids, const omm_paged_kv* kv,
                       int32_t group_size, float scale, const omm_view4* out, float* lse,
                       int32_t epoch, void* stream, const GateArgs& gate) {
  int rc = check_q_out("omm_sel_fwd_paged", q, out);
  if (rc) return rc;
  OMM_REQUIRE(ids != nullptr && kv != nullptr, OMM_EINVAL, "omm_sel_fwd_paged: null argument");
  OMM_REQUIRE(group_size >= 1, OMM_EINVAL, "omm_sel_fwd_paged: group_size must be >= 1");
  const int64_t MG = cdiv64(q->size[1], group_size);
  OMM_REQUIRE(ids->size[0] == q->size[0] && ids->size[1] == MG && ids->size[2] == q->size[2] &&
                  ids->size[3] >= 1,
              OMM_EINVAL, "omm_sel_fwd_paged: block_indices must be [B, %lld, H, T]", (long long)MG);
  OMM_REQUIRE(kv->head_dim == q->size[3] && kv->num_heads == q->size[2], OMM_EINVAL,
              "omm_sel_fwd_paged: cache geometry (H=%d, D=%d) does not match q", kv->num_heads,
              kv->head_dim);
  OMM_REQUIRE(kv->page_tokens >= 1 && kv->chunk_len >= 1 &&
                  kv->pages_per_chunk == cdiv64(kv->chunk_len, kv->page_tokens) &&
                  kv->unit_table != nullptr,
              OMM_EINVAL, "omm_sel_fwd_paged: inconsistent cache geometry");
  OMM_REQUIRE(kv->stage_map_epoch == nullptr ||
                  (kv->stage_map_slot != nullptr && kv->stage_k != nullptr &&
                   kv->stage_v != nullptr &&
                   (kv->dtype != OMM_FP8E4M3 ||
                    (kv->stage_scale_k != nullptr && kv->stage_scale_v != nullptr))),
              OMM_EINVAL, "omm_sel_fwd_paged: incomplete staging pool");
  Geom gm;
  rc = geom(*q, MG, ids->size[3], group_size, gm);
  if (rc) return rc;
  if (gm.items == 0) return OMM_OK;
  OMM_REQUIRE(ids_offsets_fit32(*ids), OMM_EUNSUPPORTED,
              "omm_sel_fwd_paged: ids must span fewer than 2^31 elements");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool mfma = qo_mfma_ok(*q, *out) && kv->head_dim % 64 == 0;
  const int32_t* idp = static_cast<const int32_t*>(ids->data);
  if (kv->dtype == OMM_BF16) {
    PagedAcc<bf16_t> acc{static_cast<const bf16_t*>(kv->pool_k), static_cast<const bf16_t*>(kv->pool_v),
                         nullptr, nullptr, static_cast<const bf16_t*>(kv->host_k),
                         static_cast<const bf16_t*>(kv->host_v), nullptr, nullptr, kv->unit_table,
                         idp, kv->stamp, kv->reads, kv->page_seen, kv->touches,
                         static_cast<const bf16_t*>(kv->stage_k),
                         static_cast<const bf16_t*>(kv->stage_v), nullptr, nullptr,
                         kv->stage_map_epoch, kv->stage_map_slot, ids->stride[0],
                         ids->stride[1], ids->stride[2],
                         ids->stride[3], kv->max_chunks, kv->n_chunks, kv->chunk_len,
                         kv->page_tokens, kv->pages_per_chunk, kv->head_dim, epoch,
                         kv->n_slots, kv->n_host_slots};
    return dispatch<bf16_t>(gm, *q, *out, lse, acc, 1, scale, mfma, 1, 2 * kv->head_dim, s, gate);
  }
  if (kv->dtype == OMM_FP8E4M3) {
    OMM_REQUIRE(kv->scale_k != nullptr && kv->scale_v != nullptr, OMM_EINVAL,
                "omm_sel_fwd_paged: fp8 cache without scales");
    PagedAcc<uint8_t> acc{static_cast<const uint8_t*>(kv->pool_k), static_cast<const uint8_t*>(kv->pool_v),
                          kv->scale_k, kv->scale_v, static_cast<const uint8_t*>(kv->host_k),
                          static_cast<const uint8_t*>(kv->host_v), kv->host_scale_k,
                          kv->host_scale_v, kv->unit_table, idp, kv->stamp, kv->reads, kv->page_seen,
                          kv->touches, static_cast<const uint8_t*>(kv->stage_k),
                          static_cast<const uint8_t*>(kv->stage_v), kv->stage_scale_k,
                          kv->stage_scale_v, kv->stage_map_epoch, kv->stage_map_slot,
                          ids->stride[0],
                          ids->stride[1], ids->stride[2], ids->stride[3], kv->max_chunks,
                          kv->n_chunks, kv->chunk_len, kv->page_tokens, kv->pages_per_chunk,
                          kv->head_dim, epoch, kv->n_slots, kv->n_host_slots};
    if (kv->qk_fp8) {
      OMM_REQUIRE(mfma && scale != 0.0f && __builtin_isfinite(scale) &&
                      (kv->head_dim == 64 || kv->head_dim == 128),
                  OMM_EUNSUPPORTED,
                  "omm_sel_fwd_paged: the fp8 QK^T variant needs head dim 64 or 128, 16-byte q / "
                  "out rows and a finite non-zero scale");
      return kv->head_dim == 128 ? launch_qk8<PagedAcc<uint8_t>, 128>(gm, *q, *out, lse, acc, 1, scale, s, gate)
                                 : launch_qk8<PagedAcc<uint8_t>, 64>(gm, *q, *out, lse, acc, 1, scale, s, gate);
    }
    return dispatch<bf16_t>(gm, *q, *out, lse, acc, 1, scale, mfma, 1, 2 * kv->head_dim, s, gate);
  }
  return set_error(OMM_EINVAL, "omm_sel_fwd_paged: unsupported cache dtype %d", kv->dtype);
}
}  // namespace
}  // namespace omm

extern "C" int omm_sel_fwd_paged(const omm_view4* q, const omm_view4* ids, const omm_paged_kv* kv,
                                 int32_t group_size, float scale, const omm_view4* out, float* lse,
                                 int32_t epoch, void* stream) {
  return omm::sel_fwd_paged_impl(q, ids, kv, group_size, scale, out, lse, epoch, stream,
                                 omm::GateArgs{});
}

extern "C" int omm_sel_fwd_paged_gated(const omm_view4* q, const omm_view4* ids,
                                       const omm_paged_kv* kv, int32_t group_size, float scale,
                                       const omm_view4* gates, const omm_view4* o_cmp,
                                       const omm_view4* o_swa, const omm_view4* out, float* lse,
                                       int32_t epoch, void* stream) {
  using namespace omm;
  OMM_REQUIRE(kv != nullptr, OMM_EINVAL, "omm_sel_fwd_paged_gated: null argument");
  // the bf16 epilogue reads each element before the same thread writes it, so the identical view
  // is safe there; the fp8 cache's first pass writes out before the mix pass reads the branches
  GateArgs ga;
  const int rc = gate_args("omm_sel_fwd_paged_gated", q, gates, o_cmp, o_swa, out,
                           kv->dtype == OMM_BF16, ga);
  if (rc) return rc;
  return sel_fwd_paged_impl(q, ids, kv, group_size, scale, out, lse, epoch, stream, ga);
}
