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
    pool_rows_kernel<T><<<grid, 64, 0, stream>>>(static_cast<const T*>(x.data), x.stride[0],
                                                 x.stride[1], static_cast<T*>(const_cast<void*>(out.data)),
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
