// Device building blocks shared by the selection-attention forward and backward kernels:
// MFMA wrappers, block accessors (dense, reference pointer tables, paged cache), the per-wave
// block walk, and the gfx950 global -> LDS copy helpers.
#pragma once

#include "omm_common.h"

namespace omm {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  __device__ __forceinline__ static f32x4 run(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    return pack_bf16x2(lo, hi);
  }
};
template <> struct Mfma<f16_t> {
  __device__ __forceinline__ static f32x4 run(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    const _Float16 a = static_cast<_Float16>(lo), b = static_cast<_Float16>(hi);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
  }
};

// e4m3 x e4m3 -> fp32, 16 x 16 x 32: lane l holds A row l % 16 and B column l % 16, k = 8 (l / 16)
// .. + 7 as 8 bytes (the 16x16x32 bf16 layout with 8-bit elements); products are exact in fp32.
__device__ __forceinline__ f32x4 mfma_fp8(uint2 a, uint2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(__builtin_bit_cast(long, a),
                                                    __builtin_bit_cast(long, b), c, 0, 0, 0);
}

// 8 packed bf16 -> 8 floats (exact)
__device__ __forceinline__ void unpack_bf16x8_sel(const uint4& r, float (&f)[8]) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
  }
}

// Optional gate combine in the attention epilogue (the NSA branch mix): out = g[0] * o_cmp +
// g[1] * o_slc + g[2] * o_swa per (query, head), fp32 arithmetic and one rounding; g == nullptr
// writes o_slc alone.  Gates bf16 [B, M, H, 3] and the branch outputs bf16 [B, M, H, D] (unit
// dim stride), element strides.
struct GateArgs {
  const bf16_t* g = nullptr;
  int64_t gs0 = 0, gs1 = 0, gs2 = 0, gs3 = 0;
  const bf16_t* oc = nullptr;
  int64_t cs0 = 0, cs1 = 0, cs2 = 0;
  const bf16_t* ow = nullptr;
  int64_t ws0 = 0, ws1 = 0, ws2 = 0;
};

// One lane's 4 consecutive output dims (d0 .. d0 + 3) of query (b, m, h): o4 = o_slc (fp32,
// normalised) -> the gated mix packed as 4 bf16.
__device__ __forceinline__ uint2 gate_mix4(const GateArgs& ga, int b, int m, int h, int d0,
                                           const float (&o4)[4]) {
  const uint16_t* gp = reinterpret_cast<const uint16_t*>(ga.g + b * ga.gs0 + m * ga.gs1 + h * ga.gs2);
  const float g0 = bf16_bits_to_f32(gp[0]), g1 = bf16_bits_to_f32(gp[ga.gs3]);
  const float g2 = bf16_bits_to_f32(gp[2 * ga.gs3]);
  const uint2 c = *reinterpret_cast<const uint2*>(ga.oc + b * ga.cs0 + m * ga.cs1 + h * ga.cs2 + d0);
  const uint2 w = *reinterpret_cast<const uint2*>(ga.ow + b * ga.ws0 + m * ga.ws1 + h * ga.ws2 + d0);
  const uint32_t cw[2] = {c.x, c.y}, ww[2] = {w.x, w.y};
  float r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t cb = e & 1 ? cw[e >> 1] & 0xffff0000u : cw[e >> 1] << 16;
    const uint32_t wb = e & 1 ? ww[e >> 1] & 0xffff0000u : ww[e >> 1] << 16;
    r[e] = __builtin_fmaf(g2, __builtin_bit_cast(float, wb),
                          __builtin_fmaf(g1, o4[e], g0 * __builtin_bit_cast(float, cb)));
  }
  return make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]));
}

// ---- block accessors ---------------------------------------------------------------------
// A resolved block: nvalid tokens visible from row 0, rows at k + r*sk (elements of its storage
// type), k == nullptr when the block is skipped.
struct BlockRef {
  const void* k;
  const void* v;
  int64_t sk, sv;
  int nvalid;
  float scale_k, scale_v;
};

// Each accessor resolves slot t of a row in two steps: resolve() -> a compact entry (Ent: a few
// 32-bit words, n = visible tokens, n <= 0 when skipped), evaluated by the MFMA kernels for 64
// slots at once, one per lane; ref() -> the block's addresses from a wave-uniform entry.
// order_key() orders the blocks of a row by position in memory (the walk visits them in that
// order, so concurrent rows that share blocks tend to read them at the same time).
// Slot t of row (b, g, h) of an ids view, as a 32-bit element offset: the (b, g, h) part is
// wave-uniform (scalar arithmetic), the lane's t part one 32-bit multiply.  The host checks
// ids_offsets_fit32 before it builds an accessor that uses this.
__device__ __forceinline__ int ids_off32(int64_t is0, int64_t is1, int64_t is2, int64_t is3,
                                         int b, int g, int h, int t) {
  return static_cast<int32_t>(b * is0 + g * is1 + h * is2) + t * static_cast<int32_t>(is3);
}

inline bool ids_offsets_fit32(const omm_view4& ids) {
  int64_t last = 0;
  for (int i = 0; i < 4; ++i) {
    if (ids.stride[i] < 0 || ids.stride[i] > 2147483647ll) return false;
    if (ids.size[i] > 0) last += (ids.size[i] - 1) * ids.stride[i];
  }
  return last < 2147483647ll;
}

// DenseAcc::ref forms token offsets in 32 bits: (N - 1) * the token stride of k and v below 2^32
// elements, strides non-negative.
inline bool kv_offsets_fit32(const omm_view4& k, const omm_view4& v) {
  for (const omm_view4* x : {&k, &v}) {
    if (x->stride[1] < 0) return false;
    if (x->size[1] > 0 && (x->size[1] - 1) * x->stride[1] >= (int64_t{1} << 32)) return false;
  }
  return true;
}

template <typename T>
struct DenseAcc {
  static constexpr bool kMayMisalign = false;  // 16-byte rows checked on the host
  using KV = T;
  struct Ent {
    int t0, n;  // first token, visible tokens
  };
  View4<const T> k, v;
  const int32_t* ids;
  int64_t is0, is1, is2, is3;
  int N, bs, chunk;
  bool causal;
  __device__ __forceinline__ Ent resolve(int b, int g, int h, int t, int q_chunk) const {
    Ent e{0, 0};
    const int32_t bid = ids[ids_off32(is0, is1, is2, is3, b, g, h, t)];
    if (bid < 0) return e;
    const int64_t t0 = static_cast<int64_t>(bid) * bs;
    if (t0 >= N) return e;
    int64_t n = N - t0 < bs ? N - t0 : bs;
    if (causal) {
      // visible prefix ends at the query chunk's end: t0 / chunk > q_chunk  <=>  lim <= 0
      const int64_t lim = static_cast<int64_t>(q_chunk + 1) * chunk - t0;
      n = n < lim ? n : lim;
    }
    if (n <= 0) return e;
    e.t0 = static_cast<int>(t0);
    e.n = static_cast<int>(n);
    return e;
  }
  // the (b, h) slice's base in 64 bits, the token offset in 32 (the host keeps every slice's
  // token extent under 2^32 elements: kv_offsets_fit32), so no 64-bit multiply per block
  __device__ __forceinline__ BlockRef ref(int b, int h, const Ent& e) const {
    const T* kb = k.p + (static_cast<int64_t>(b) * k.s0 + static_cast<int64_t>(h) * k.s2);
    const T* vb = v.p + (static_cast<int64_t>(b) * v.s0 + static_cast<int64_t>(h) * v.s2);
    const uint32_t ko = static_cast<uint32_t>(e.t0) * static_cast<uint32_t>(k.s1);
    const uint32_t vo = static_cast<uint32_t>(e.t0) * static_cast<uint32_t>(v.s1);
    return BlockRef{kb + ko, vb + vo, k.s1, v.s1, e.n, 1.0f, 1.0f};
  }
  __device__ __forceinline__ static int64_t order_key(const Ent& e) { return e.t0; }
  __device__ __forceinline__ void touch(int, int, int, int) const {}
};

struct PtrAcc {
  using KV = bf16_t;
  // raw caller addresses: any 2-byte alignment is accepted (the reference's contract), so the
  // staging checks each block and copies misaligned ones with 2-byte loads
  static constexpr bool kMayMisalign = true;
  struct Ent {
    int64_t k, v;  // raw addresses (0 = skip)
    int n;
    int pad;
  };
  const int64_t* pk;
  const int64_t* pv;
  int64_t s0, s1, s2, s3;
  int64_t stride_n;
  int bs;
  __device__ __forceinline__ Ent resolve(int b, int g, int h, int t, int) const {
    const int64_t off = b * s0 + g * s1 + h * s2 + t * s3;
    Ent e{pk[off], pv[off], 0, 0};
    e.n = (e.k == 0 || e.v == 0) ? 0 : bs;
    return e;
  }
  __device__ __forceinline__ BlockRef ref(int, int, const Ent& e) const {
    return BlockRef{reinterpret_cast<const void*>(static_cast<uintptr_t>(e.k)),
                    reinterpret_cast<const void*>(static_cast<uintptr_t>(e.v)), stride_n,
                    stride_n, e.n, 1.0f, 1.0f};
  }
  __device__ __forceinline__ static int64_t order_key(const Ent& e) { return e.k; }
  __device__ __forceinline__ void touch(int, int, int, int) const {}
};

// Paged entries: page >= 0 is an HBM pool page, page < 0 the host pool page -1 - page; bid is
// the block id (the walk order must not depend on residency); fp8 pages carry their
// dequantisation scales.
struct PagedEnt16 {
  int page, n, bid;
};
struct PagedEnt8 {
  int page, n, bid;
  float sk, sv;
};
template <typename KVT> struct PagedEntOf { using type = PagedEnt16; };
template <> struct PagedEntOf<uint8_t> { using type = PagedEnt8; };

template <typename KVT>
struct PagedAcc {
  static constexpr bool kMayMisalign = false;  // 16-byte rows checked on the host
  using KV = KVT;
  using Ent = typename PagedEntOf<KVT>::type;
  const KVT* pool_k;
  const KVT* pool_v;
  const float* sc_k;
  const float* sc_v;
  const KVT* host_k;
  const KVT* host_v;
  const float* hsc_k;
  const float* hsc_v;
  const int32_t* unit;
  const int32_t* ids;
  int32_t* stamp;
  int32_t* reads;
  uint8_t* seen;
  int32_t* touches;
  // staged host pages (omm_paged_stage under this epoch), or smap_epoch == nullptr
  const KVT* stage_k;
  const KVT* stage_v;
  const float* ssc_k;
  const float* ssc_v;
  const int32_t* smap_epoch;
  const int32_t* smap_slot;
  int64_t is0, is1, is2, is3;
  int max_chunks, n_chunks, chunk_len, P, ppc, D, epoch, n_slots, n_host;
  // Ent::page: >= 0 page of the HBM pool, kStaged | slot a staging-pool slot, < 0 page
  // -1 - page of the host pool
  static constexpr int kStaged = 1 << 30;
  __device__ __forceinline__ Ent resolve(int b, int g, int h, int t, int) const {
    Ent e{};
    const int32_t bid = ids[ids_off32(is0, is1, is2, is3, b, g, h, t)];
    if (bid < 0) return e;
    const int cid = bid / ppc, p = bid - cid * ppc;
    if (cid >= n_chunks || cid >= max_chunks) return e;
    const int32_t s = unit[static_cast<int64_t>(h) * max_chunks + cid];
    if (s == -1 || s >= n_slots || (s < 0 && -2 - s >= n_host)) return e;
    const int page = (s >= 0 ? s : -2 - s) * ppc + p;
    const int rem = chunk_len - p * P;
    e.page = s >= 0 ? page : -1 - page;
    e.n = rem < P ? rem : P;
    e.bid = bid;
    int ss = -1;
    if (s < 0 && smap_epoch != nullptr && epoch > 0) {
      const int64_t mi = (static_cast<int64_t>(h) * max_chunks + cid) * ppc + p;
      if (smap_epoch[mi] == epoch) ss = smap_slot[mi];
      if (ss >= 0) e.page = kStaged | ss;
    }
    if constexpr (sizeof(KVT) == 1) {
      const float* ck = ss >= 0 ? ssc_k : (s >= 0 ? sc_k : hsc_k);
      const float* cv = ss >= 0 ? ssc_v : (s >= 0 ? sc_v : hsc_v);
      const int pi = ss >= 0 ? ss : page;
      e.sk = ck != nullptr ? ck[pi] : 1.0f;
      e.sv = cv != nullptr ? cv[pi] : 1.0f;
    }
    return e;
  }
  __device__ __forceinline__ BlockRef ref(int, int, const Ent& e) const {
    const bool hbm = e.page >= 0;
    const bool staged = e.page >= kStaged;
    const int64_t off =
        static_cast<int64_t>(staged ? e.page - kStaged : (hbm ? e.page : -1 - e.page)) * P * D;
    const KVT* bk = staged ? stage_k : (hbm ? pool_k : host_k);
    const KVT* bv = staged ? stage_v : (hbm ? pool_v : host_v);
    BlockRef r{bk + off, bv + off, D, D, e.n, 1.0f, 1.0f};
    if constexpr (sizeof(KVT) == 1) {
      r.scale_k = e.sk;
      r.scale_v = e.sv;
    }
    return r;
  }
  __device__ __forceinline__ static int64_t order_key(const Ent& e) { return e.bid; }
  // LRU touch: stamp every readable unit this workgroup's row lists (duplicates store the same
  // epoch, so the races are benign), count its pages read (vector atomics) and mark each listed
  // page seen (duplicates store the same 1).  With touches, the stamp is exchanged atomically and
  // the one lane of the whole call that moves it to this epoch counts the unit's access.
  __device__ __forceinline__ void touch(int b, int g, int h, int T) const {
    const bool st = stamp != nullptr && epoch > 0;
    if (!st && reads == nullptr && seen == nullptr) return;
    for (int t = threadIdx.x; t < T; t += blockDim.x) {
      const int32_t bid = ids[b * is0 + g * is1 + h * is2 + t * is3];
      if (bid < 0) continue;
      const int cid = bid / ppc;
      if (cid >= n_chunks || cid >= max_chunks) continue;
      const int64_t u = static_cast<int64_t>(h) * max_chunks + cid;
      if (unit[u] == -1) continue;
      if (st && touches != nullptr) {
        if (atomicExch(stamp + u, epoch) != epoch) atomicAdd(touches + u, 1);
      } else if (st) {
        stamp[u] = epoch;
      }
      if (reads != nullptr) atomicAdd(reads + u, 1);
      if (seen != nullptr) seen[u * ppc + (bid - cid * ppc)] = 1;
    }
  }
};

template <typename Acc>
__device__ __forceinline__ BlockRef resolve_block(const Acc& acc, int b, int g, int h, int t,
                                                  int qc) {
  const typename Acc::Ent e = acc.resolve(b, g, h, t, qc);
  if (e.n <= 0) return BlockRef{nullptr, nullptr, 0, 0, 0, 1.0f, 1.0f};
  return acc.ref(b, h, e);
}

// Key tiles of up to 64 tokens over the listed blocks (wave-uniform), one slot at a time.
struct TileIt {
  int t, tok0, n;  // block slot, first token of the tile within the block, tokens in tile
  BlockRef br;
  bool valid;
};

template <typename Acc>
__device__ __forceinline__ TileIt first_tile(const Acc& acc, int b, int g, int h, int T, int qc,
                                             int t) {
  TileIt it;
  for (; t < T; ++t) {
    const BlockRef br = resolve_block(acc, b, g, h, t, qc);
    if (br.k != nullptr && br.nvalid > 0) {
      it.t = t;
      it.tok0 = 0;
      it.br = br;
      it.n = br.nvalid < 64 ? br.nvalid : 64;
      it.valid = true;
      return it;
    }
  }
  it.valid = false;
  it.t = T;
  it.tok0 = 0;
  it.n = 0;
  it.br = BlockRef{nullptr, nullptr, 0, 0, 0, 1.0f, 1.0f};
  return it;
}

template <typename Acc>
__device__ __forceinline__ TileIt next_tile(const Acc& acc, const TileIt& c, int b, int g, int h,
                                            int T, int qc) {
  if (c.tok0 + 64 < c.br.nvalid) {
    TileIt it = c;
    it.tok0 += 64;
    const int rem = c.br.nvalid - it.tok0;
    it.n = rem < 64 ? rem : 64;
    return it;
  }
  return first_tile(acc, b, g, h, T, qc, c.t + 1);
}


// Element i of a K / V block in fp32 (fp8 pages: the dequantised value the MFMA path sees).
template <typename KVT> __device__ __forceinline__ float kv_elem(const void* p, int64_t i, float s);
template <> __device__ __forceinline__ float kv_elem<float>(const void* p, int64_t i, float) {
  return static_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float kv_elem<bf16_t>(const void* p, int64_t i, float) {
  return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <> __device__ __forceinline__ float kv_elem<f16_t>(const void* p, int64_t i, float) {
  return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}
template <> __device__ __forceinline__ float kv_elem<uint8_t>(const void* p, int64_t i, float s) {
  // the dequantised value the MFMA path computes with: code * page scale in fp32
  return e4m3_to_f32(static_cast<const uint8_t*>(p)[i]) * s;
}

// The same walk for a wave that resolved 64 slots at once: lane i holds the entry of slot
// base + i.  Live slots are visited in ascending order_key (ties by slot): every workgroup then
// sweeps its blocks from low to high addresses, so the workgroups running together on an XCD
// read overlapping blocks at about the same time and share them in L2.  A slot's rank among the
// live slots is counted once per 64 slots (one readlane and compare per live slot); the next
// block is then a compare, a ballot and a find-first-set, with no memory access.  Within a row
// the order only changes the fp32 summation order of the softmax.
template <typename E>
__device__ __forceinline__ E lane_entry(const E& e, int lane) {
  static_assert(sizeof(E) % 4 == 0, "entries are 32-bit words");
  constexpr int W = sizeof(E) / 4;
  int w[W];
  __builtin_memcpy(w, &e, sizeof(E));
#pragma unroll
  for (int i = 0; i < W; ++i) w[i] = __builtin_amdgcn_readlane(w[i], lane);
  E r;
  __builtin_memcpy(&r, w, sizeof(E));
  return r;
}

template <typename Acc, int TK = 64>
struct WaveWalk {
  typename Acc::Ent e;
  int rank;        // this lane's rank among the live slots of the batch (-1: not live)
  int nlive, pos;  // live slots in the batch; rank of the current block (-1 before the first)
  int base;        // first slot of the batch
  int tok0, n;     // current tile: first token within the block, tokens (<= TK)
  BlockRef br;
  bool valid;

  __device__ __forceinline__ void fill(const Acc& acc, int b, int g, int h, int T, int qc) {
    const int lane = lane_id();
    const int t = base + lane;
    if (t < T) {
      e = acc.resolve(b, g, h, t, qc);
    } else {
      e = typename Acc::Ent{};
    }
    const bool live = e.n > 0;
    uint64_t m = __ballot(live);
    nlive = __builtin_popcountll(m);
    const int64_t key = Acc::order_key(e);
    int r = 0;
    while (m != 0ull) {
      const int l = __builtin_ctzll(m);
      m &= m - 1ull;
      const int64_t ko = static_cast<int64_t>(
          (static_cast<uint64_t>(static_cast<uint32_t>(
               __builtin_amdgcn_readlane(static_cast<int>(key >> 32), l))) << 32) |
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), l)));
      r += (ko < key || (ko == key && l < lane)) ? 1 : 0;
    }
    rank = live ? r : -1;
    pos = -1;
  }
  // advance to the first tile of the next live slot
  __device__ __forceinline__ void next_block(const Acc& acc, int b, int g, int h, int T, int qc) {
    for (;;) {
      if (pos + 1 < nlive) {
        ++pos;
        const int slot = __builtin_ctzll(__ballot(rank == pos));
        br = acc.ref(b, h, lane_entry(e, slot));
        tok0 = 0;
        n = br.nvalid < TK ? br.nvalid : TK;
        valid = true;
        return;
      }
      base += 64;
      if (base >= T) {
        valid = false;
        n = 0;
        return;
      }
      fill(acc, b, g, h, T, qc);
    }
  }
  __device__ __forceinline__ void start(const Acc& acc, int b, int g, int h, int T, int qc) {
    start_at(acc, b, g, h, 0, T, qc);
  }
  // walk only the slots [lo, hi) of the row (advance() then takes hi as its T)
  __device__ __forceinline__ void start_at(const Acc& acc, int b, int g, int h, int lo, int hi,
                                           int qc) {
    base = lo;
    valid = false;
    if (hi <= lo) return;
    fill(acc, b, g, h, hi, qc);
    next_block(acc, b, g, h, hi, qc);
  }
  __device__ __forceinline__ void advance(const Acc& acc, int b, int g, int h, int T, int qc) {
    if (tok0 + TK < br.nvalid) {
      tok0 += TK;
      const int rem = br.nvalid - tok0;
      n = rem < TK ? rem : TK;
      return;
    }
    next_block(acc, b, g, h, T, qc);
  }
};

// ---- gfx950 LDS copies ------------------------------------------------------------------------
// K / V (or Q / dO) tiles of 8 KiB: TK rows of D 16-bit elements, copied global -> LDS by
// buffer_load ... lds, 16-byte chunk c of row r stored at chunk slot c ^ swz(r).
template <int D>
struct DmaGeom {
  static constexpr int ROWB = 2 * D;       // bytes per K / V row
  static constexpr int CPR = D / 8;        // 16-byte chunks per row
  static constexpr int TK = 8192 / ROWB;   // keys per tile
  static constexpr int RPI = 1024 / ROWB;  // rows per copy instruction (64 lanes x 16 bytes)
  static constexpr int NT = TK / 16;       // 16-key score blocks per tile
  static constexpr int NU = TK / 32;       // 32-key PV steps per tile
  static constexpr int SD = D / 32;        // QK k-steps
  static constexpr int ND = D / 16;        // PV d-tiles
  __device__ static int swz_k(int r) { return r & (CPR - 1); }
  __device__ static int swz_v(int r) { return ((r & 7) << 1) & (CPR - 1); }
};

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
#define OMM_LDS(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  const bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (__attribute__((address_space(3))) bf16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer descriptor (gfx9 layout): base address, stride 0, num_records = nbytes (loads at or
// past it read 0), dword 3 = the gfx9 data-format bits of an untyped buffer.
__device__ __forceinline__ i32x4 buffer_desc(const void* base, int nbytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32));  // address bits 32-47
  r.z = __builtin_amdgcn_readfirstlane(nbytes);
  r.w = 0x00020000;
  return r;
}

// This wave's NI of the 8 copy instructions of one K or V tile (NI = 8 / waves per workgroup):
// rows [0, nrows) of `base` (row stride rsb bytes) into the 8 KiB LDS buffer dst; instruction
// j (= NI w + jj) fills dst bytes [1024 j, 1024 j + 1024) and off[jj] is this lane's source
// offset for it.  Issued as inline asm (M0 = LDS destination): the compiler then does not treat
// it as an LDS store, so it does not make the next LDS read wait for this copy; the kernel
// orders copies and reads itself (s_waitcnt vmcnt(0) and a barrier before a buffer is read, a
// barrier before it is refilled).  M0 is set here and used by nothing else in the kernel.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int NI>
__device__ __forceinline__ void dma_part(const void* base, int rsb, int nrows, char* dst, int w,
                                         const int (&off)[NI]) {
  static_assert(NI == 2 || NI == 4, "2 or 4 copy instructions per wave");
  const i32x4 r = buffer_desc(base, nrows * rsb);
  const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst)) + 1024u * NI * w)));
  if constexpr (NI == 4) {
    asm volatile(
        "s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %5, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 0x400\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %5, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 0x400\n\ts_nop 0\n\tbuffer_load_dwordx4 %3, %5, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 0x400\n\ts_nop 0\n\tbuffer_load_dwordx4 %4, %5, 0 offen lds"
        :
        : "s"(m0), "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(r)
        : "memory", "m0", "scc");
  } else {
    asm volatile(
        "s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
        "s_add_u32 m0, m0, 0x400\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds"
        :
        : "s"(m0), "v"(off[0]), "v"(off[1]), "s"(r)
        : "memory", "m0", "scc");
  }
}
#pragma clang diagnostic pop

// dma_part's copy for a block whose address is not 16-byte aligned: the same LDS bytes (rows past
// nrows as 0), through 2-byte loads and ordinary LDS stores.
template <int NI>
__device__ __forceinline__ void copy_part_u16(const void* base, int rsb, int nrows, char* dst,
                                              int w, const int (&off)[NI]) {
  const int lim = nrows * rsb;
  const int lane = lane_id();
#pragma unroll
  for (int jj = 0; jj < NI; ++jj) {
    uint32_t wd[4] = {0u, 0u, 0u, 0u};
    if (off[jj] < lim) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(static_cast<const char*>(base) + off[jj]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        wd[i] = static_cast<uint32_t>(p[2 * i]) | (static_cast<uint32_t>(p[2 * i + 1]) << 16);
    }
    *reinterpret_cast<uint4*>(dst + 1024 * (NI * w + jj) + 16 * lane) =
        make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }
}

// One wave's part of a K or V tile copy: LDS DMA, or the 2-byte copy for a misaligned block of an
// accessor that admits them (wave-uniform test; every wave of the workgroup copies the same block).
template <typename Acc, int NI>
__device__ __forceinline__ void copy_part(const void* base, int rsb, int nrows, char* dst, int w,
                                          const int (&off)[NI]) {
  if constexpr (Acc::kMayMisalign) {
    if ((reinterpret_cast<uintptr_t>(base) & 15u) != 0u) {
      copy_part_u16<NI>(base, rsb, nrows, dst, w, off);
      return;
    }
  }
  dma_part<NI>(base, rsb, nrows, dst, w, off);
}

}  // namespace
}  // namespace omm
