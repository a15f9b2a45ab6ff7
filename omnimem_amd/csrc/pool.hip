// Block compression (mean-pooled key blocks) and query-group pooling.
// out[b, j, h, :] = mean of x[b, t, h, :] over t in [j*group, min((j+1)*group, T)), computed as
// an fp32 sum in ascending t, one IEEE division by the count, one RNE rounding to T.
// Reference: models/transformers/causal_wan_nsa_model.py:408 (K pool), nsa/ops/index_topk.py:76
// (query-group pool); both are torch `.mean` in the input dtype.
#include "omm_common.h"

namespace omm {
namespace {

template <typename T> struct Vec16;
template <> struct Vec16<bf16_t> { static constexpr int N = 8; };
template <> struct Vec16<f16_t> { static constexpr int N = 8; };
template <> struct Vec16<float> { static constexpr int N = 4; };

template <typename T>
__device__ __forceinline__ void unpack16(const uint4& r, float (&f)[Vec16<T>::N]) {
  const T* e = reinterpret_cast<const T*>(&r);
#pragma unroll
  for (int i = 0; i < Vec16<T>::N; ++i) f[i] = to_f32<T>(e[i]);
}

// Token rows with a contiguous (H, D) plane: each lane owns 16 bytes of the plane.
template <typename T>
__global__ __launch_bounds__(64) void pool_rows_kernel(const T* __restrict__ x, int64_t xs0,
                                                        int64_t xs1, T* __restrict__ out,
                                                        int64_t os0, int64_t os1, int T_len,
                                                        int HD, int group) {
  constexpr int V = Vec16<T>::N;
  const int col = (static_cast<int>(blockIdx.x) * 64 + lane_id()) * V;
  if (col >= HD) return;
  const int j = blockIdx.y, b = blockIdx.z;
  const int t0 = j * group;
  const int t1 = min(t0 + group, T_len);
  const T* base = x + b * xs0 + col;
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  int t = t0;
  constexpr int U = 8;
  for (; t + U <= t1; t += U) {
    uint4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      r[u] = *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(t + u) * xs1);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float f[V];
      unpack16<T>(r[u], f);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += f[i];
    }
  }
  for (; t < t1; ++t) {
    const uint4 r = *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(t) * xs1);
    float f[V];
    unpack16<T>(r, f);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] += f[i];
  }
  const float cnt = static_cast<float>(t1 - t0);
  T res[V];
#pragma unroll
  for (int i = 0; i < V; ++i) res[i] = from_f32<T>(acc[i] / cnt);
  *reinterpret_cast<uint4*>(out + b * os0 + static_cast<int64_t>(j) * os1 + col) =
      *reinterpret_cast<const uint4*>(res);
}

// The same pooling with 4 waves per (64 lanes x 16 bytes of the plane, row j), for launches that
// hold few one-wave workgroups: wave w loads tokens 16 w .. 16 w + 15 of each 64-token run into
// LDS, then adds 4-byte word w of every staged 16-byte column, element by element in token order,
// so the sums are those of pool_rows_kernel.  AR chunk q (222 workgroups): 4.4 against 5.9 us.
constexpr int kPoolRowsWaves = 4;

template <typename T>
__global__ __launch_bounds__(kPoolRowsWaves * kWave) void pool_rows_wg_kernel(
    const T* __restrict__ x, int64_t xs0, int64_t xs1, T* __restrict__ out, int64_t os0,
    int64_t os1, int T_len, int HD, int group) {
  constexpr int V = Vec16<T>::N;
  constexpr int E = V / kPoolRowsWaves;       // elements of a 4-byte word
  constexpr int RW = kWave / kPoolRowsWaves;  // rows per wave per run
  __shared__ uint4 st[kWave][kWave];          // [token of the run][lane]
  const int w = static_cast<int>(threadIdx.x) / kWave, lane = lane_id();
  const int col = (static_cast<int>(blockIdx.x) * kWave + lane) * V;
  const bool ok = col < HD;
  const int j = blockIdx.y, b = blockIdx.z;
  const int t0 = j * group;
  const int t1 = min(t0 + group, T_len);
  const T* base = x + b * xs0 + (ok ? col : 0);
  float acc[E];
#pragma unroll
  for (int i = 0; i < E; ++i) acc[i] = 0.0f;
  for (int c0 = t0; c0 < t1; c0 += kWave) {  // workgroup-uniform
    const int n = min(kWave, t1 - c0);
    uint4 r[RW];
#pragma unroll
    for (int u = 0; u < RW; ++u) {
      const int row = RW * w + u;
      r[u] = (ok && row < n) ? *reinterpret_cast<const uint4*>(base + static_cast<int64_t>(c0 + row) * xs1)
                             : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < RW; ++u) st[RW * w + u][lane] = r[u];
    __syncthreads();
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&st[0][lane]) + w;
    for (int row = 0; row < n; ++row) {
      const uint32_t word = src[row * kWave * 4];
      const T* e = reinterpret_cast<const T*>(&word);
#pragma unroll
      for (int i = 0; i < E; ++i) acc[i] += to_f32<T>(e[i]);
    }
    __syncthreads();
  }
  if (!ok) return;
  const float cnt = static_cast<float>(t1 - t0);
  T* dst = out + b * os0 + static_cast<int64_t>(j) * os1 + col + E * w;
#pragma unroll
  for (int i = 0; i < E; ++i) dst[i] = from_f32<T>(acc[i] / cnt);
}

// Any strides: one thread per output element.
template <typename T>
__global__ __launch_bounds__(256) void pool_generic_kernel(View4<const T> x, View4<T> out, int B,
                                                           int MG, int H, int D, int T_len,
                                                           int group) {
  const int64_t total = static_cast<int64_t>(B) * MG * H * D;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int d = static_cast<int>(i % D);
    const int h = static_cast<int>((i / D) % H);
    const int j = static_cast<int>((i / (static_cast<int64_t>(D) * H)) % MG);
    const int b = static_cast<int>(i / (static_cast<int64_t>(D) * H * MG));
    const int t0 = j * group, t1 = min(t0 + group, T_len);
    float acc = 0.0f;
    for (int t = t0; t < t1; ++t) acc += to_f32<T>(*x.at(b, t, h, d));
    *out.at(b, j, h, d) = from_f32<T>(acc / static_cast<float>(t1 - t0));
  }
}

template <typename T>
int launch_pool(const omm_view4& x, const omm_view4& out, int group, hipStream_t stream) {
  const int B = static_cast<int>(x.size[0]), T_len = static_cast<int>(x.size[1]);
  const int H = static_cast<int>(x.size[2]), D = static_cast<int>(x.size[3]);
  const int MG = static_cast<int>(cdiv64(T_len, group));
  constexpr int V = Vec16<T>::N;
  const int HD = H * D;
  const bool rows_ok = x.stride[3] == 1 && x.stride[2] == D && out.stride[3] == 1 &&
                       out.stride[2] == D && HD % V == 0 && x.stride[1] % V == 0 &&
                       x.stride[0] % V == 0 && out.stride[1] % V == 0 && out.stride[0] % V == 0 &&
                       (reinterpret_cast<uintptr_t>(x.data) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(out.data) & 15u) == 0;
  if (rows_ok) {
    const dim3 grid(static_cast<unsigned>(cdiv64(HD, 64 * V)), static_cast<unsigned>(MG),
                    static_cast<unsigned>(B));
    const T* xp = static_cast<const T*>(x.data);
    T* op = static_cast<T*>(const_cast<void*>(out.data));
    if (static_cast<int64_t>(grid.x) * grid.y * grid.z < 1024)  // fewer than 4 waves per CU
      pool_rows_wg_kernel<T><<<grid, kPoolRowsWaves * kWave, 0, stream>>>(
          xp, x.stride[0], x.stride[1], op, out.stride[0], out.stride[1], T_len, HD, group);
    else
      pool_rows_kernel<T><<<grid, 64, 0, stream>>>(xp, x.stride[0], x.stride[1], op,
                                                   out.stride[0], out.stride[1], T_len, HD, group);
  } else {
    const int64_t total = static_cast<int64_t>(B) * MG * H * D;
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(cdiv64(total, 256), 65535));
    pool_generic_kernel<T><<<blocks, 256, 0, stream>>>(make_view<const T>(x), make_view<T>(out), B,
                                                       MG, H, D, T_len, group);
  }
  return check_launch("omm_block_pool");
}

}  // namespace

int pool_launch(const omm_view4& x, const omm_view4& out, int32_t dtype, int group,
                hipStream_t stream) {
  switch (dtype) {
    case OMM_F32: return launch_pool<float>(x, out, group, stream);
    case OMM_BF16: return launch_pool<bf16_t>(x, out, group, stream);
    case OMM_F16: return launch_pool<f16_t>(x, out, group, stream);
    default: return set_error(OMM_EINVAL, "block pool: unsupported dtype %d", dtype);
  }
}

}  // namespace omm

extern "C" int omm_block_pool(const omm_view4* x, const omm_view4* out, int32_t dtype,
                              int32_t group, void* stream) {
  using namespace omm;
  OMM_REQUIRE(x != nullptr && out != nullptr, OMM_EINVAL, "omm_block_pool: null view");
  OMM_REQUIRE(group >= 1, OMM_EINVAL, "omm_block_pool: group must be >= 1, got %d", group);
  for (int i = 0; i < 4; ++i)
    OMM_REQUIRE(x->size[i] >= 0 && x->stride[i] >= 0 && out->stride[i] >= 0, OMM_EINVAL,
                "omm_block_pool: negative size or stride");
  const int64_t MG = cdiv64(x->size[1], group);
  OMM_REQUIRE(out->size[0] == x->size[0] && out->size[1] == MG && out->size[2] == x->size[2] &&
                  out->size[3] == x->size[3],
              OMM_EINVAL, "omm_block_pool: out must be [%lld, %lld, %lld, %lld]",
              (long long)x->size[0], (long long)MG, (long long)x->size[2], (long long)x->size[3]);
  OMM_REQUIRE(x->size[0] * MG * x->size[2] * x->size[3] < (1ll << 40), OMM_EINVAL,
              "omm_block_pool: tensor too large");
  OMM_REQUIRE(MG <= 65535 && x->size[0] <= 65535, OMM_EUNSUPPORTED,
              "omm_block_pool: grid limit (blocks %lld, batch %lld)", (long long)MG,
              (long long)x->size[0]);
  if (x->size[0] == 0 || x->size[1] == 0 || x->size[2] == 0 || x->size[3] == 0) return OMM_OK;
  OMM_REQUIRE(x->data != nullptr && out->data != nullptr, OMM_EINVAL, "omm_block_pool: null data");
  return pool_launch(*x, *out, dtype, group, static_cast<hipStream_t>(stream));
}
