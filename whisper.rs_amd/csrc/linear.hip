// Projections with f16 weights: out(t, r) = W[r] . x[t] + bias[r]
// (replaces crates/tensor/src/ops/quant.rs:415-473 f16_linear, reached through
//  LinearWeight::linear, crates/tensor/src/weight.rs:116-137, from the
//  encoder's fused QKV projection, crates/whisper/src/encoder.rs:275-277, and
//  the cross-attention K/V precompute, crates/whisper/src/decoder.rs:423-447).
//
// K6 (linear_f16w): D^T = W X^T on v_mfma_f32_32x32x16_f16. Both operands are
//   "k-contiguous" rows as stored (W [n_out][n_in] f16, X [n_tokens][k] f16),
//   so neither needs a transpose. A workgroup of 4 waves owns a tile of 128
//   output features x 128 tokens; wave (wm, wn) owns 64 x 64 of it as 2 x 2
//   MFMA tiles. k advances 64 per LDS stage: the next stage's global loads are
//   in flight in registers while the current stage's MFMAs run, then land in
//   the other LDS buffer; one barrier per stage. LDS rows (128 bytes) keep
//   their 16-byte chunks XOR-permuted by the row index, so the 32 rows read
//   by one operand fetch spread over the banks.
//   f32 activations are made exact on the f16 matrix pipe by a pre-pass
//   (linear_split_rows): each row is scaled by a power of two so that its
//   largest element lies in [2^14, 2^15), then split into three f16 parts
//   hi + mid + lo that sum to it (parts below 2^-24 of the row maximum are
//   dropped). The GEMM then runs over k' = 3 n_in with the weight column
//   k' mod n_in, so every product is exact and only the f32 accumulation
//   rounds, as in dot_f16_f32 (simd.rs:593-700). The epilogue multiplies by
//   the row's 2^-shift (exact), adds the f32 bias and stores 4 consecutive
//   features per lane in the output type, at
//   out + t * out_rs + (r / 64) * out_hs + r % 64: token-major rows
//   (out_hs = 64) or the arena's [head][token][64] planes.
#include "wrs_internal.hpp"

namespace wrs {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 128;  // output features per workgroup (MFMA M)
constexpr int kBN = 128;  // tokens per workgroup (MFMA N)
constexpr int kBK = kLinearK;  // k per LDS stage (64)
constexpr int kChunks = kBK / 8;  // 16-byte chunks per tile row
constexpr int kLoads = kBM * kChunks / kThreads;  // 16-byte loads per thread per operand

static_assert(kBM == kBN, "one load pattern serves both operands");
static_assert(kChunks == 8, "the chunk swizzle assumes 8 chunks per row");

__device__ inline int swz(int row, int chunk) { return chunk ^ (row & 7); }

template <typename OutT>
__device__ inline void store4(OutT* p, const f32x4& v);
template <>
__device__ inline void store4<float>(float* p, const f32x4& v) {
  *reinterpret_cast<f32x4*>(p) = v;
}
template <>
__device__ inline void store4<_Float16>(_Float16* p, const f32x4& v) {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  const f16x4 h = __builtin_convertvector(v, f16x4);
  *reinterpret_cast<u32x2*>(p) = __builtin_bit_cast(u32x2, h);
}
template <>
__device__ inline void store4<__bf16>(__bf16* p, const f32x4& v) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  const bf16x4 h = __builtin_convertvector(v, bf16x4);
  *reinterpret_cast<u32x2*>(p) = __builtin_bit_cast(u32x2, h);
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void linear_f16w(LinearArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 lds_a[2][kBM * kBK];
  __shared__ __attribute__((aligned(16))) _Float16 lds_b[2][kBN * kBK];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.x * kBM;  // first output feature
  const int n0 = blockIdx.y * kBN;  // first token
  const int grp = blockIdx.z;
  const _Float16* w = a.w[grp];

  // Global -> register loads of one stage: thread tid moves chunks tid + 256 i.
  // Rows past the matrix edge read the last row (their results are dropped).
  const _Float16* ga[kLoads];
  const _Float16* gb[kLoads];
  int lofs[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int c = tid + kThreads * i;
    const int row = c / kChunks, ch = c % kChunks;
    const int ra = min(m0 + row, a.n_out - 1);
    const int rb = min(n0 + row, a.n_tokens - 1);
    ga[i] = w + static_cast<int64_t>(ra) * a.n_in + ch * 8;
    gb[i] = a.x + static_cast<int64_t>(rb) * a.x_rs + ch * 8;
    lofs[i] = row * kBK + swz(row, ch) * 8;
  }
  u32x4 ra_[kLoads], rb_[kLoads];
  auto load_stage = [&](int kt) {
    const int kx = kt * kBK;        // column of x' (k' space)
    const int kw = kx % a.n_in;     // column of W
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      ra_[i] = *reinterpret_cast<const u32x4*>(ga[i] + kw);
      rb_[i] = *reinterpret_cast<const u32x4*>(gb[i] + kx);
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      *reinterpret_cast<u32x4*>(&lds_a[buf][lofs[i]]) = ra_[i];
      *reinterpret_cast<u32x4*>(&lds_b[buf][lofs[i]]) = rb_[i];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Operand rows of this lane: feature/token l % 32 of each 32-row MFMA tile,
  // k-group l / 32 (8 consecutive k) of each 16-k step.
  const int orow = lane & 31, kgrp = lane >> 5;
  const int n_kt = a.k_total / kBK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < n_kt) load_stage(kt + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int ch = 2 * ks + kgrp;
      f16x8 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int ra = wm * 64 + i * 32 + orow;
        av[i] = *reinterpret_cast<const f16x8*>(&lds_a[buf][ra * kBK + swz(ra, ch) * 8]);
        const int rb = wn * 64 + i * 32 + orow;
        bv[i] = *reinterpret_cast<const f16x8*>(&lds_b[buf][rb * kBK + swz(rb, ch) * 8]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < n_kt) {
      store_stage(buf ^ 1);  // that buffer was last read before the previous barrier
      __syncthreads();
    }
  }

  // Epilogue: acc[i][j][e] is feature m0 + 64 wm + 32 i + 8 (e / 4) + 4 kgrp + e % 4
  // of token n0 + 64 wn + 32 j + orow.
  OutT* out = reinterpret_cast<OutT*>(a.out[grp]);
  const float* bias = a.bias[grp];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = n0 + wn * 64 + j * 32 + orow;
    if (t >= a.n_tokens) continue;
    const float rs = a.row_scale ? a.row_scale[t] : 1.0f;
    OutT* orow_p = out + static_cast<int64_t>(t) * a.out_rs;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = m0 + wm * 64 + i * 32 + 8 * g + 4 * kgrp;
        if (r >= a.n_out) continue;
        f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                   acc[i][j][4 * g + 3]};
        v *= rs;
        if (bias) v += *reinterpret_cast<const f32x4*>(bias + r);
        store4<OutT>(orow_p + static_cast<int64_t>(r >> 6) * a.out_hs + (r & 63), v);
      }
  }
}

// f32 rows -> [hi | mid | lo] f16 rows of 3 n_in, plus each row's 2^-shift.
// One wave per row.
__device__ inline float pow2(int e) { return __builtin_bit_cast(float, (e + 127) << 23); }
__device__ inline int clamp_exp(int e) { return e < -126 ? -126 : (e > 127 ? 127 : e); }

__global__ __launch_bounds__(256) void linear_split_rows(const float* x, int64_t x_rs,
                                                         int n_tokens, int n_in,
                                                         _Float16* xs, float* row_scale) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= n_tokens) return;
  const float* xr = x + static_cast<int64_t>(t) * x_rs;
  float amax = 0.0f;
  for (int k = lane; k < n_in; k += 64) amax = fmaxf(amax, fabsf(xr[k]));
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const int e_max = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xFF);
  const int sh = e_max == 0 ? 0 : clamp_exp(141 - e_max);
  const float up = pow2(sh);
  _Float16* dst = xs + static_cast<int64_t>(t) * 3 * n_in;
  for (int k = lane; k < n_in; k += 64) {
    const float v = xr[k] * up;
    const _Float16 h = static_cast<_Float16>(v);
    const float r1 = v - static_cast<float>(h);
    const _Float16 m = static_cast<_Float16>(r1);
    dst[k] = h;
    dst[n_in + k] = m;
    dst[2 * n_in + k] = static_cast<_Float16>(r1 - static_cast<float>(m));
  }
  if (lane == 0) row_scale[t] = pow2(clamp_exp(-sh));
}

}  // namespace

hipError_t launch_linear_split(const float* x, int64_t x_rs, int n_tokens, int n_in,
                               _Float16* xs, float* row_scale, hipStream_t s) {
  if (n_tokens <= 0) return hipSuccess;
  hipLaunchKernelGGL(linear_split_rows, dim3((n_tokens + 3) / 4), dim3(256), 0, s, x, x_rs,
                     n_tokens, n_in, xs, row_scale);
  return hipGetLastError();
}

hipError_t launch_linear_f16w(const LinearArgs& a, DType out_dt, hipStream_t s) {
  if (a.n_tokens <= 0 || a.n_out <= 0 || a.n_groups <= 0) return hipSuccess;
  dim3 grid((a.n_out + kBM - 1) / kBM, (a.n_tokens + kBN - 1) / kBN, a.n_groups);
  switch (out_dt) {
    case kF32: hipLaunchKernelGGL(linear_f16w<float>, grid, dim3(kThreads), 0, s, a); break;
    case kF16: hipLaunchKernelGGL(linear_f16w<_Float16>, grid, dim3(kThreads), 0, s, a); break;
    case kBF16: hipLaunchKernelGGL(linear_f16w<__bf16>, grid, dim3(kThreads), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace wrs
