// Shared device/host helpers for the gfx950 selection-path kernels.
// Element strides everywhere; fp32 accumulation; wave64 (CDNA4) execution.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>

#include "../../include/omnimem_hip.h"

namespace omm {

constexpr int kWave = 64;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- error plumbing (host) ------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Device fill by a kernel (graph-capture safe, unlike a memset node).
int fill_i32(int32_t* p, int64_t n, int32_t value, hipStream_t stream);
// Mean pooling of runs of `group` tokens (omm_block_pool without argument checks).
int pool_launch(const omm_view4& x, const omm_view4& out, int32_t dtype, int group,
                hipStream_t stream);

#define OMM_REQUIRE(cond, code, ...) \
  do {                               \
    if (!(cond)) return ::omm::set_error((code), __VA_ARGS__); \
  } while (0)

inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Whether the byte spans of two views of elem-byte elements intersect (empty views never do;
// negative strides widen the span downwards).
inline bool views_overlap(const omm_view4& a, const omm_view4& b, int64_t elem) {
  auto span = [elem](const omm_view4& v, intptr_t& lo, intptr_t& hi) {
    lo = hi = reinterpret_cast<intptr_t>(v.data);
    for (int i = 0; i < 4; ++i) {
      if (v.size[i] <= 0) return false;
      const int64_t ext = (v.size[i] - 1) * v.stride[i] * elem;
      (ext < 0 ? lo : hi) += ext;
    }
    hi += elem;
    return true;
  };
  intptr_t alo, ahi, blo, bhi;
  if (!span(a, alo, ahi) || !span(b, blo, bhi)) return false;
  return alo < bhi && blo < ahi;
}

// ---- scalar conversions (device + host) -------------------------------------------------
__host__ __device__ inline float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}
// Round-to-nearest-even, quiet NaN preserved.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  const uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(r >> 16);
}

// OCP fp8 e4m3fn (bias 7, no inf, 0x7f = NaN, max 448).  Round-to-nearest-even, saturating.
__host__ __device__ inline uint8_t f32_to_e4m3(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint8_t sign = static_cast<uint8_t>((u >> 24) & 0x80u);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint8_t>(sign | 0x7f);
  const float a = __builtin_bit_cast(float, u & 0x7fffffffu);
  int code;
  if (a < 0.015625f) {  // below the smallest normal 2^-6: multiples of 2^-9
    code = static_cast<int>(__builtin_rintf(a * 512.0f));
  } else if (a >= 480.0f) {
    code = 0x7e;
  } else {
    const int e = static_cast<int>((__builtin_bit_cast(uint32_t, a) >> 23) & 0xffu) - 127;
    // a * 2^(3-e) is exact (power-of-two scaling of a normal float into [8, 16))
    const float m = a * __builtin_bit_cast(float, static_cast<uint32_t>(127 + 3 - e) << 23);
    code = ((e + 7) << 3) + static_cast<int>(__builtin_rintf(m)) - 8;
  }
  if (code > 0x7e) code = 0x7e;
  return static_cast<uint8_t>(sign | code);
}
__host__ __device__ inline float e4m3_to_f32(uint8_t c) {
  const uint32_t sign = static_cast<uint32_t>(c & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  if ((c & 0x7fu) == 0x7fu) return __builtin_bit_cast(float, 0x7fc00000u | sign);
  float v;
  if (e == 0) {
    v = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  } else {
    v = static_cast<float>(8u + m) * __builtin_bit_cast(float, (e - 10u + 127u) << 23);
  }
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) | sign);
}

// ---- hardware conversions (gfx950) ------------------------------------------------------------
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 omm_bf16x2;

// Two floats -> packed bf16 pair (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const omm_bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}
// Eight OCP e4m3fn codes (byte 0 first) -> eight bf16 (v_cvt_scalef32_pk_bf16_fp8 with scale 1:
// exact; every e4m3 value is a bf16 value).
__device__ __forceinline__ uint4 e4m3x8_to_bf16(uint2 c) {
  const omm_bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.x, 1.0f, false);
  const omm_bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.x, 1.0f, true);
  const omm_bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.y, 1.0f, false);
  const omm_bf16x2 e = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.y, 1.0f, true);
  return make_uint4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                    __builtin_bit_cast(uint32_t, d), __builtin_bit_cast(uint32_t, e));
}
// Four floats already within [-448, 448] -> four e4m3fn codes, round to nearest even
// (v_cvt_pk_fp8_f32).
__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return static_cast<uint32_t>(w);
}

// Element traits: T is the storage type of q/k/v tensors.
struct bf16_t { uint16_t bits; };
struct f16_t { _Float16 v; };

template <typename T> struct Elem;
template <> struct Elem<float> {
  __host__ __device__ static float load(float x) { return x; }
  __host__ __device__ static float store(float x) { return x; }
};
template <> struct Elem<bf16_t> {
  __host__ __device__ static float load(bf16_t x) { return bf16_bits_to_f32(x.bits); }
  __host__ __device__ static bf16_t store(float x) { return bf16_t{f32_to_bf16_bits(x)}; }
};
template <> struct Elem<f16_t> {
  __host__ __device__ static float load(f16_t x) { return static_cast<float>(x.v); }
  __host__ __device__ static f16_t store(float x) { return f16_t{static_cast<_Float16>(x)}; }
};

template <typename T> __host__ __device__ inline float to_f32(T x) { return Elem<T>::load(x); }
template <typename T> __host__ __device__ inline T from_f32(float x) { return Elem<T>::store(x); }

// ---- strided views ------------------------------------------------------------------------
template <typename T>
struct View4 {
  T* p;
  int64_t s0, s1, s2, s3;
  __device__ __forceinline__ T* at(int64_t i0, int64_t i1, int64_t i2, int64_t i3 = 0) const {
    return p + i0 * s0 + i1 * s1 + i2 * s2 + i3 * s3;
  }
};
template <typename T>
inline View4<T> make_view(const omm_view4& v) {
  return View4<T>{static_cast<T*>(const_cast<void*>(v.data)), v.stride[0], v.stride[1],
                  v.stride[2], v.stride[3]};
}

// ---- top-k keys -----------------------------------------------------------------------------
// Order-preserving float -> uint32 (+0 and -0 map to the same code, as the reference's float
// comparison treats them as equal); key = ord << 32 | (NC-1-id) so that a larger key means
// (score desc, id asc).  0 is reserved for "no candidate".
__device__ __forceinline__ uint32_t f32_ord(float f) {
  f = (f == 0.0f) ? 0.0f : f;
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint64_t make_key(float s, int c, int nc) {
  // -inf and NaN are never selected.
  if (!(s > kNegInf)) return 0ull;
  return (static_cast<uint64_t>(f32_ord(s)) << 32) | static_cast<uint32_t>(nc - 1 - c);
}
__device__ __forceinline__ int key_id(uint64_t key, int nc) {
  return nc - 1 - static_cast<int>(static_cast<uint32_t>(key));
}

// ---- wave64 helpers -------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ float wave_max_xor(float v, int lo_mask, int hi_mask) {
  for (int m = lo_mask; m <= hi_mask; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Bitonic sort of one uint64 per lane across the wave, descending (lane 0 = largest).
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t x) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint64_t o = shfl_xor_u64(x, j);
      const bool want_max = (((lane & k) == 0) == ((lane & j) == 0));
      x = want_max ? (x > o ? x : o) : (x < o ? x : o);
    }
  }
  return x;
}

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }
__device__ __forceinline__ int popc64(uint64_t m) { return __builtin_popcountll(m); }
// Number of set bits of m in lanes below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  const int lane = lane_id();
  const uint64_t below = (lane == 0) ? 0ull : (m & ((1ull << lane) - 1ull));
  return __builtin_popcountll(below);
}

// XCD-aware workgroup order: the dispatcher hands consecutive workgroup ids to the 8 XCDs in
// turn, so id -> (id % 8) * per + id / 8 gives every XCD one contiguous range of work items
// (and its own L2 the matching slice of K/V).  Ids past 8 * per map to themselves.
__device__ __forceinline__ int xcd_remap(int id, int total) {
  constexpr int kXcd = 8;
  const int per = total / kXcd;
  if (id >= per * kXcd) return id;
  return (id % kXcd) * per + id / kXcd;
}

}  // namespace omm
