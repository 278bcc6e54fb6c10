// Decode-step attention: one new query row per beam / slot against cached K/V.
//
// K2 (decode_f16): split-K attention over the f16 KV cache
//   (replaces crates/tensor/src/ops/attention.rs:246-434 single_token_mha_d64
//    as called from crates/whisper/src/decoder.rs:636 / :698).
//   Grid (split, head, group). A workgroup owns `chunk` = 64 consecutive keys
//   of one (group, head) plane and ALL query rows of the group (the beams of
//   an utterance share the cross-attention plane, so it is read once per step
//   instead of once per beam). Each thread issues its K and V loads (2 x 16 B
//   each) before any arithmetic, so the whole layer's cache is in flight from
//   the first cycle. Partial (max, sum, acc[64]) per row go to scratch; the
//   last workgroup of a (group, head) to finish -- detected with an
//   agent-scope counter -- merges them with the log-sum-exp rule and writes
//   the output, then re-arms the counter for the next launch.
//
// decode_exact_f32: the reference's own decode arithmetic on f32 K/V for the
//   host-slice entry points: full score row, max, exp, sum, reciprocal
//   multiply (softmax.rs:1-23), weights below 1e-7 skipped (attention.rs:366,
//   decoder.rs:884). Row i of a call sees keys [0, row_limit0 + i).
#include "wrs_internal.hpp"

namespace wrs {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kChunk = 64;  // keys per workgroup (4 threads per key)
constexpr int kPart = 66;   // floats per partial row: m, l, acc[64]

__device__ inline float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

template <int R>
__global__ __launch_bounds__(kThreads) void decode_f16(DecodeArgs a) {
  __shared__ float qs[R][64];
  __shared__ float ps[R][kChunk];
  __shared__ __attribute__((aligned(16))) _Float16 vs[kChunk][64 + 8];
  __shared__ float red[4][R][64];
  __shared__ float mrow[R], lrow[R];
  __shared__ int last_flag;

  const int split = blockIdx.x, h = blockIdx.y, g = blockIdx.z;
  const int tid = threadIdx.x;
  const int rows = a.rows_per_group;
  const int len = a.len[g];
  const int k_lo = split * kChunk;

  // Issue every cache load of this workgroup first.
  const int kl = tid >> 2, part = tid & 3;
  const int key = k_lo + kl;
  const bool valid = key < len;
  const _Float16* kp = a.k + a.goff[g] + h * a.kv_hs + static_cast<int64_t>(key) * 64 + part * 16;
  const _Float16* vp = a.v + a.goff[g] + h * a.kv_hs + static_cast<int64_t>(key) * 64 + part * 16;
  u32x4 k0 = {0, 0, 0, 0}, k1 = {0, 0, 0, 0}, v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
  if (valid) {
    k0 = *reinterpret_cast<const u32x4*>(kp);
    k1 = *reinterpret_cast<const u32x4*>(kp + 8);
    v0 = *reinterpret_cast<const u32x4*>(vp);
    v1 = *reinterpret_cast<const u32x4*>(vp + 8);
  }

  // Queries of the group, pre-scaled so scores come out in the exp2 domain.
  for (int e = tid; e < R * 64; e += kThreads) {
    const int r = e >> 6, d = e & 63;
    float x = 0.f;
    if (r < rows)
      x = a.q[static_cast<int64_t>(g * rows + r) * a.q_rs + h * 64 + d] * a.scale_log2;
    qs[r][d] = x;
  }
  __syncthreads();

  // Scores: 16-wide partial dot per thread, reduced over the 4 threads of a key.
  {
    const f16x8 ka = __builtin_bit_cast(f16x8, k0);
    const f16x8 kb = __builtin_bit_cast(f16x8, k1);
    float kf[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      kf[i] = static_cast<float>(ka[i]);
      kf[8 + i] = static_cast<float>(kb[i]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) s = __builtin_fmaf(qs[r][part * 16 + i], kf[i], s);
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      if (part == 0) ps[r][kl] = valid ? s : -INFINITY;
    }
  }
  *reinterpret_cast<u32x4*>(&vs[kl][part * 16]) = v0;
  *reinterpret_cast<u32x4*>(&vs[kl][part * 16 + 8]) = v1;
  __syncthreads();

  // Softmax statistics of this chunk: one wave per row.
  const int wave = tid >> 6, lane = tid & 63;
  for (int r = wave; r < R; r += 4) {
    const float x = ps[r][lane];
    const float mx = wave_max(x);
    const float p = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(x - mx);
    const float sum = wave_sum(p);
    ps[r][lane] = p;
    if (lane == 0) {
      mrow[r] = mx;
      lrow[r] = sum;
    }
  }
  __syncthreads();

  // P V over the chunk: thread (quarter, d) sums 16 keys for every row.
  {
    const int d = tid & 63, qq = tid >> 6;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kk = qq * 16 + i;
      const float vv = static_cast<float>(vs[kk][d]);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = __builtin_fmaf(ps[r][kk], vv, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) red[qq][r][d] = acc[r];
  }
  __syncthreads();

  if (a.n_splits == 1) {
    // Whole row in one workgroup: normalize and store directly.
    for (int e = tid; e < rows * 64; e += kThreads) {
      const int r = e >> 6, d = e & 63;
      const float v = red[0][r][d] + red[1][r][d] + red[2][r][d] + red[3][r][d];
      const float l = lrow[r];
      a.o[static_cast<int64_t>(g * rows + r) * a.o_rs + h * 64 + d] = l > 0.f ? v * (1.f / l) : 0.f;
    }
    return;
  }

  const int gh = g * a.n_heads + h;
  float* mine = a.part + (static_cast<int64_t>(gh) * a.n_splits + split) * rows * kPart;
  for (int e = tid; e < rows * 64; e += kThreads) {
    const int r = e >> 6, d = e & 63;
    mine[r * kPart + 2 + d] = red[0][r][d] + red[1][r][d] + red[2][r][d] + red[3][r][d];
  }
  if (tid < rows) {
    mine[tid * kPart] = mrow[tid];
    mine[tid * kPart + 1] = lrow[tid];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned done = atomicAdd(a.counters + gh, 1u);
    last_flag = (done == static_cast<unsigned>(a.n_splits - 1));
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();

  // Log-sum-exp merge of all splits (values are in the exp2 domain).
  const float* base = a.part + static_cast<int64_t>(gh) * a.n_splits * rows * kPart;
  for (int e = tid; e < rows * 64; e += kThreads) {
    const int r = e >> 6, d = e & 63;
    float M = -INFINITY;
    for (int sp = 0; sp < a.n_splits; ++sp) M = fmaxf(M, base[(sp * rows + r) * kPart]);
    float L = 0.f, acc = 0.f;
    for (int sp = 0; sp < a.n_splits; ++sp) {
      const float* pr = base + (sp * rows + r) * kPart;
      const float ms = pr[0];
      const float w = (ms == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms - M);
      L = __builtin_fmaf(pr[1], w, L);
      acc = __builtin_fmaf(pr[2 + d], w, acc);
    }
    a.o[static_cast<int64_t>(g * rows + r) * a.o_rs + h * 64 + d] = L > 0.f ? acc * (1.f / L) : 0.f;
  }
  if (tid == 0) a.counters[gh] = 0u;
}

__device__ inline float block_reduce(float x, float* sh, bool is_max) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  x = is_max ? wave_max(x) : wave_sum(x);
  __syncthreads();
  if (lane == 0) sh[wave] = x;
  __syncthreads();
  float r = sh[0];
  for (int w = 1; w < kThreads / 64; ++w) r = is_max ? fmaxf(r, sh[w]) : r + sh[w];
  return r;
}

__global__ __launch_bounds__(kThreads) void decode_exact_f32(ExactArgs a) {
  __shared__ float qsh[128];
  __shared__ float sh[kThreads / 64];
  __shared__ float accs[4][128];
  const int h = blockIdx.x, row = blockIdx.y;
  const int tid = threadIdx.x;
  const int dh = a.d_head;
  const float* q = a.q + static_cast<int64_t>(row) * a.q_rs + h * dh;
  for (int d = tid; d < dh; d += kThreads) qsh[d] = q[d];
  __syncthreads();

  const int L = a.row_limit0 + row;
  float* sc = a.scores + (static_cast<int64_t>(row) * a.n_heads + h) * a.scores_stride;
  float lmax = -INFINITY;
  for (int j = tid; j < L; j += kThreads) {
    const float* kr = a.k + static_cast<int64_t>(j) * a.kv_rs + h * dh;
    float dot = 0.f;
    for (int d = 0; d < dh; ++d) dot = __builtin_fmaf(qsh[d], kr[d], dot);
    const float s = dot * a.scale;
    sc[j] = s;
    lmax = fmaxf(lmax, s);
  }
  const float mx = block_reduce(lmax, sh, true);
  float lsum = 0.f;
  for (int j = tid; j < L; j += kThreads) {
    const float p = expf(sc[j] - mx);
    sc[j] = p;
    lsum += p;
  }
  const float sum = block_reduce(lsum, sh, false);
  const float inv = 1.f / sum;

  // Weighted values, weights below 1e-7 skipped. Thread (quarter, d).
  const int qq = tid >> 6, dl = tid & 63;
  for (int d0 = 0; d0 < dh; d0 += 64) {
    const int d = d0 + dl;
    float acc = 0.f;
    if (d < dh) {
      for (int j = qq; j < L; j += 4) {
        const float w = sc[j] * inv;
        if (w < 1e-7f) continue;
        acc = __builtin_fmaf(w, a.v[static_cast<int64_t>(j) * a.kv_rs + h * dh + d], acc);
      }
    }
    accs[qq][dl] = acc;
    __syncthreads();
    if (qq == 0 && d < dh)
      a.o[static_cast<int64_t>(row) * a.o_rs + h * dh + d] =
          accs[0][dl] + accs[1][dl] + accs[2][dl] + accs[3][dl];
    __syncthreads();
  }
}

}  // namespace

size_t decode_part_floats(int n_groups, int n_heads, int n_splits, int rows) {
  return static_cast<size_t>(n_groups) * n_heads * n_splits * rows * kPart;
}

hipError_t launch_decode_f16(const DecodeArgs& a, hipStream_t s) {
  if (a.n_groups <= 0 || a.n_splits <= 0) return hipSuccess;
  const dim3 grid(a.n_splits, a.n_heads, a.n_groups), block(kThreads);
  switch (a.rows_per_group) {
    case 1: hipLaunchKernelGGL(decode_f16<1>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(decode_f16<2>, grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL(decode_f16<3>, grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL(decode_f16<4>, grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL(decode_f16<5>, grid, block, 0, s, a); break;
    case 6: hipLaunchKernelGGL(decode_f16<6>, grid, block, 0, s, a); break;
    case 7: hipLaunchKernelGGL(decode_f16<7>, grid, block, 0, s, a); break;
    case 8: hipLaunchKernelGGL(decode_f16<8>, grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode_exact_f32(const ExactArgs& a, hipStream_t s) {
  if (a.n_rows <= 0 || a.n_heads <= 0) return hipSuccess;
  const dim3 grid(a.n_heads, a.n_rows), block(kThreads);
  hipLaunchKernelGGL(decode_exact_f32, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace wrs
