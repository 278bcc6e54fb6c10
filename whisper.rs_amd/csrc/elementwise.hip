// Row and element kernels around the projections of a Whisper block.
//
// K8 (layer_norm_rows): LayerNorm over rows of d_model f32 values
//   (replaces crates/tensor/src/ops/norm.rs:116-143, called at
//   crates/whisper/src/encoder.rs:266-274 and decoder.rs:586-594, :660-668,
//   :737-745). One wave per row: mean, then the variance around it, each a
//   sum of per-lane float4 partials reduced with DPP and two cross-row moves;
//   inv_std = 1 / sqrt(var + eps); out = fma((x - mean) * inv_std, gamma, beta)
//   as norm.rs:53-57 forms it, stored as f32 or rounded to f16 / bf16 for a
//   following projection. Rows of up to 2048 values are held in registers
//   between the three passes (one read); longer rows are re-read from L1.
//
// K9 (gelu_f32): GELU, tanh form (crates/tensor/src/ops/gelu.rs:6-23, called
//   at decoder.rs:753 and in the encoder MLP), in place on f32, the reference's
//   order of operations with contraction off; four values per thread.
#include "wrs_internal.hpp"

#include <algorithm>

namespace wrs {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                0xF, 0xF, false));
}
__device__ inline float wave_sum64(float v) {
  v += dpp<0xB1>(v);   // xor 1
  v += dpp<0x4E>(v);   // xor 2
  v += dpp<0x141>(v);  // mirror in each half row of 8
  v += dpp<0x140>(v);  // mirror in each row of 16
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

template <typename OutT>
__device__ inline void store4(OutT* p, const f32x4& v);
template <>
__device__ inline void store4<float>(float* p, const f32x4& v) {
  *reinterpret_cast<f32x4*>(p) = v;
}
template <>
__device__ inline void store4<_Float16>(_Float16* p, const f32x4& v) {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  *reinterpret_cast<u32x2*>(p) = __builtin_bit_cast(u32x2, __builtin_convertvector(v, f16x4));
}
template <>
__device__ inline void store4<__bf16>(__bf16* p, const f32x4& v) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  *reinterpret_cast<u32x2*>(p) = __builtin_bit_cast(u32x2, __builtin_convertvector(v, bf16x4));
}

constexpr int kLnWaves = 4;

// kCached > 0: the row (at most 256 kCached values) is held in registers and
// read once; kCached == 0 reads it again for the variance and the output.
template <typename OutT, int kCached>
__global__ __launch_bounds__(64 * kLnWaves) void layer_norm_rows(const float* x,
                                                                 const float* gamma,
                                                                 const float* beta, float eps,
                                                                 int n_tokens, int d, OutT* out) {
  const int row = blockIdx.x * kLnWaves + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n_tokens) return;  // whole wave
  const float* xr = x + static_cast<int64_t>(row) * d;
  OutT* orow = out + static_cast<int64_t>(row) * d;
  if constexpr (kCached > 0) {
    // The row, gamma and beta are all requested before the reductions.
    f32x4 v[kCached], gv[kCached], bv[kCached];
#pragma unroll
    for (int i = 0; i < kCached; ++i) {
      const int k = 4 * lane + 256 * i;
      const bool in = k < d;
      v[i] = in ? *reinterpret_cast<const f32x4*>(xr + k) : f32x4{0.f, 0.f, 0.f, 0.f};
      gv[i] = in ? *reinterpret_cast<const f32x4*>(gamma + k) : f32x4{0.f, 0.f, 0.f, 0.f};
      bv[i] = in ? *reinterpret_cast<const f32x4*>(beta + k) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kCached; ++i) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
    const float mean = wave_sum64(s) / static_cast<float>(d);
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < kCached; ++i) {
      if (4 * lane + 256 * i >= d) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) q = fmaf(v[i][j] - mean, v[i][j] - mean, q);
    }
    const float var = wave_sum64(q) / static_cast<float>(d);
    const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < kCached; ++i) {
      const int k = 4 * lane + 256 * i;
      if (k >= d) break;
      f32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = fmaf((v[i][j] - mean) * inv_std, gv[i][j], bv[i][j]);
      store4<OutT>(orow + k, o);
    }
    return;
  }
  float s = 0.0f;
  for (int k = 4 * lane; k < d; k += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(xr + k);
    s += (v[0] + v[1]) + (v[2] + v[3]);
  }
  const float mean = wave_sum64(s) / static_cast<float>(d);
  float q = 0.0f;
  for (int k = 4 * lane; k < d; k += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(xr + k) - mean;
#pragma unroll
    for (int j = 0; j < 4; ++j) q = fmaf(v[j], v[j], q);
  }
  const float var = wave_sum64(q) / static_cast<float>(d);
  const float inv_std = 1.0f / sqrtf(var + eps);
  for (int k = 4 * lane; k < d; k += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(xr + k);
    const f32x4 g = *reinterpret_cast<const f32x4*>(gamma + k);
    const f32x4 b = *reinterpret_cast<const f32x4*>(beta + k);
    f32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = fmaf((v[j] - mean) * inv_std, g[j], b[j]);
    store4<OutT>(orow + k, o);
  }
}

__global__ __launch_bounds__(256) void gelu_f32(float* data, int64_t n) {
  const int64_t n4 = n / 4;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n4; i += gridDim.x * 256ll) {
    f32x4 v = reinterpret_cast<f32x4*>(data)[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = gelu_tanh(v[j]);
    reinterpret_cast<f32x4*>(data)[i] = v;
  }
  for (int64_t i = 4 * n4 + blockIdx.x * 256ll + threadIdx.x; i < n; i += gridDim.x * 256ll)
    data[i] = gelu_tanh(data[i]);
}

}  // namespace

hipError_t launch_layer_norm(const float* x, const float* gamma, const float* beta, float eps,
                             int n_tokens, int d, DType out_dt, void* out, hipStream_t s) {
  if (n_tokens <= 0 || d <= 0) return hipSuccess;
  dim3 grid((n_tokens + kLnWaves - 1) / kLnWaves), block(64 * kLnWaves);
#define WRS_LN(OT)                                                                         \
  if (d <= 1280)                                                                           \
    hipLaunchKernelGGL((layer_norm_rows<OT, 5>), grid, block, 0, s, x, gamma, beta, eps,   \
                       n_tokens, d, static_cast<OT*>(out));                                \
  else if (d <= 2048)                                                                      \
    hipLaunchKernelGGL((layer_norm_rows<OT, 8>), grid, block, 0, s, x, gamma, beta, eps,   \
                       n_tokens, d, static_cast<OT*>(out));                                \
  else                                                                                     \
    hipLaunchKernelGGL((layer_norm_rows<OT, 0>), grid, block, 0, s, x, gamma, beta, eps,   \
                       n_tokens, d, static_cast<OT*>(out));
  switch (out_dt) {
    case kF32: WRS_LN(float) break;
    case kF16: WRS_LN(_Float16) break;
    case kBF16: WRS_LN(__bf16) break;
    default: return hipErrorInvalidValue;
  }
#undef WRS_LN
  return hipGetLastError();
}

hipError_t launch_gelu(float* data, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((n / 4 + 255) / 256 + 1, 4096);
  hipLaunchKernelGGL(gelu_f32, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, data, n);
  return hipGetLastError();
}

}  // namespace wrs
