// Decode-step attention: one new query row per beam / slot against cached K/V.
//
// K2 (decode_f16): split-K attention over the f16 KV cache
//   (replaces crates/tensor/src/ops/attention.rs:246-434 single_token_mha_d64
//    as called from crates/whisper/src/decoder.rs:636 / :698).
//   Grid (split, head, group). A workgroup of 1024 threads owns kChunk = 128
//   consecutive keys of one (group, head) plane and ALL query rows of the
//   group (the beams of an utterance share the cross-attention plane, so it is
//   read once per step instead of once per beam). Eight threads carry one key
//   (16 bytes of its K row and of its V row each) and issue those loads, and
//   the query loads, before any arithmetic, so the whole layer's cache is in
//   flight from the first cycles. 16 waves per workgroup (4 per SIMD) keep the
//   short score / softmax / PV phases from being bound by one wave's issue
//   rate.
//   Partials (max, sum, acc[64]) per row are published with agent-scope
//   (sc1, L2-coherent) stores; after every wave has waited for its stores, one
//   thread bumps the (group, head) counter -- each on its own 128-byte line, so
//   the increments of different heads do not serialize. The workgroup that
//   sees the last count merges all splits with the log-sum-exp rule: each of
//   its first rows*64 threads merges one output element, with the partial
//   loads of up to 16 splits in flight at once, writes the output and
//   re-arms its counter. Agent-scope atomics avoid the full-L2 writeback and
//   invalidate that a device-wide __threadfence costs on gfx950.
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
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;            // exact f32 decode
constexpr int kWgThreads = 1024;         // f16 split-K decode: 16 waves, 4 per SIMD
constexpr int kChunk = kDecodeChunk;     // keys per workgroup: one per 8 threads
constexpr int kKeyGroups = kWgThreads / 64;  // PV: 16 groups of kChunk/16 keys
constexpr int kKpl = kChunk / 64;        // softmax: keys per lane
constexpr int kPart = 68;    // floats per partial row: m, l, 2 pad, acc[64]
constexpr int kCounterStride = 32;  // 128 bytes between merge counters
constexpr int kMaxSplitsMerge = 16;  // partial loads in flight per thread in the merge

// Cross-lane moves inside a row of 16 lanes (DPP): xor 1, xor 2, mirror-8, mirror-16.
template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                0xF, 0xF, false));
}
// Sum over the 8 lanes 8i..8i+7: xor 1, xor 2 (quad perm), then row_half_mirror
// (lane 7-j of each half row of 8) adds the other quad.
__device__ inline float oct_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  return x + dpp<0x141>(x);
}
__device__ inline float wave_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ inline float wave_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

__device__ inline void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int R>
__global__ __launch_bounds__(kWgThreads) void decode_f16(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) float qs[R][64];
  __shared__ float ps[R][kChunk];
  __shared__ __attribute__((aligned(16))) _Float16 vs[kChunk][64 + 8];
  __shared__ float red[kKeyGroups][R][64];
  __shared__ float mrow[R], lrow[R];
  __shared__ int last_flag;

  const int split = blockIdx.x, h = blockIdx.y, g = blockIdx.z;
  const int tid = threadIdx.x;
  const int rows = a.rows_per_group;
  const int len = a.len[g];
  // Loads: thread (key kl, eighth pt) carries d 8*pt..8*pt+7 of one K row and
  // one V row of the chunk; threads below R*64 also carry one query element.
  const int pt = tid & 7, kl = tid >> 3;
  const int qr = tid >> 6, qd = tid & 63;
  float qv = 0.f;
  if (qr < rows)
    qv = a.q[static_cast<int64_t>(g * rows + qr) * a.q_rs + h * 64 + qd];
  const int key = split * kChunk + kl;
  const bool valid = key < len;
  u32x4 kx = {0, 0, 0, 0}, vx = {0, 0, 0, 0};
  if (valid) {
    const int64_t off = a.goff[g] + h * a.kv_hs + static_cast<int64_t>(key) * 64 + pt * 8;
    kx = *reinterpret_cast<const u32x4*>(a.k + off);
    vx = *reinterpret_cast<const u32x4*>(a.v + off);
  }
  if (qr < R) qs[qr][qd] = qv * a.scale_log2;  // rows >= `rows` hold zeros
  __syncthreads();

  // Scores in the exp2 domain: 8-wide partial dots, summed over the 8 lanes
  // of a key with DPP (xor 1, xor 2, then the 4-lane halves of the row).
  {
    const f16x8 kh = __builtin_bit_cast(f16x8, kx);
    float kf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) kf[j] = static_cast<float>(kh[j]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f32x4 q0 = *reinterpret_cast<const f32x4*>(&qs[r][pt * 8]);
      const f32x4 q1 = *reinterpret_cast<const f32x4*>(&qs[r][pt * 8 + 4]);
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) s = __builtin_fmaf(q0[j], kf[j], s);
#pragma unroll
      for (int j = 0; j < 4; ++j) s = __builtin_fmaf(q1[j], kf[4 + j], s);
      s = oct_sum(s);
      if (pt == 0) ps[r][kl] = valid ? s : -INFINITY;
    }
    *reinterpret_cast<u32x4*>(&vs[kl][pt * 8]) = vx;
  }
  __syncthreads();

  // Chunk softmax statistics: one wave per row.
  const int wave = tid >> 6, lane = tid & 63;
  if (wave < R) {
    const int r = wave;
    float x[kKpl], mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kKpl; ++i) {
      x[i] = ps[r][lane + 64 * i];
      mx = fmaxf(mx, x[i]);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kKpl; ++i) {
      const float p = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(x[i] - mx);
      ps[r][lane + 64 * i] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      mrow[r] = mx;
      lrow[r] = sum;
    }
  }
  __syncthreads();

  // P V over the chunk: thread (key group kg, d) sums 8 keys for every row.
  {
    const int d = tid & 63, kg = tid >> 6;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
    for (int i = 0; i < kChunk / kKeyGroups; ++i) {
      const int kk = kg * (kChunk / kKeyGroups) + i;
      const float vv = static_cast<float>(vs[kk][d]);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = __builtin_fmaf(ps[r][kk], vv, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) red[kg][r][d] = acc[r];
  }
  __syncthreads();

  // Thread (row qr, d qd) of the first rows*64 threads owns one output
  // element: its sum over the key groups.
  const bool own = qr < rows;
  float pv = 0.f;
  if (own) {
#pragma unroll
    for (int kg = 0; kg < kKeyGroups; ++kg) pv += red[kg][qr][qd];
  }
  if (a.n_splits == 1) {
    // The whole row in one workgroup: normalize and store directly.
    if (own) {
      const float l = lrow[qr];
      a.o[static_cast<int64_t>(g * rows + qr) * a.o_rs + h * 64 + qd] = l > 0.f ? pv * (1.f / l) : 0.f;
    }
    return;
  }

  const int gh = g * a.n_heads + h;
  float* mine = a.part + (static_cast<int64_t>(gh) * a.n_splits + split) * rows * kPart;
  if (own) st_agent(mine + qr * kPart + 4 + qd, pv);
  if (tid < rows) {
    st_agent(mine + tid * kPart, mrow[tid]);
    st_agent(mine + tid * kPart + 1, lrow[tid]);
  }
  // Every wave waits until its agent-scope stores are performed, so the
  // counter increment below is ordered after all of this workgroup's partials.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  unsigned* counter = a.counters + gh * kCounterStride;
  if (tid == 0) {
    const unsigned done = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_flag = (done == static_cast<unsigned>(a.n_splits - 1));
  }
  __syncthreads();
  if (!last_flag) return;

  // Log-sum-exp merge of all splits (exp2 domain): thread (qr, qd) merges its
  // element, issuing the partial loads of up to kMaxSplitsMerge splits at
  // once, folded online across batches of that many splits.
  if (own) {
    const float* base = a.part + static_cast<int64_t>(gh) * a.n_splits * rows * kPart;
    const int ns = a.n_splits;
    float M = -INFINITY, L = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < ns; s0 += kMaxSplitsMerge) {
      float ms[kMaxSplitsMerge], ls[kMaxSplitsMerge], as[kMaxSplitsMerge];
#pragma unroll
      for (int j = 0; j < kMaxSplitsMerge; ++j) {
        ms[j] = -INFINITY;
        ls[j] = as[j] = 0.f;
        if (s0 + j < ns) {
          const float* pr = base + ((s0 + j) * rows + qr) * kPart;
          ms[j] = ld_agent(pr);
          ls[j] = ld_agent(pr + 1);
          as[j] = ld_agent(pr + 4 + qd);
        }
      }
      float Mb = M;
#pragma unroll
      for (int j = 0; j < kMaxSplitsMerge; ++j) Mb = fmaxf(Mb, ms[j]);
      if (Mb == -INFINITY) continue;
      const float scale = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - Mb);
      L *= scale;
      acc *= scale;
#pragma unroll
      for (int j = 0; j < kMaxSplitsMerge; ++j) {
        const float w = (ms[j] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms[j] - Mb);
        L = __builtin_fmaf(ls[j], w, L);
        acc = __builtin_fmaf(as[j], w, acc);
      }
      M = Mb;
    }
    a.o[static_cast<int64_t>(g * rows + qr) * a.o_rs + h * 64 + qd] = L > 0.f ? acc * (1.f / L) : 0.f;
  }
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

size_t decode_counter_words(int n_groups, int n_heads) {
  return static_cast<size_t>(n_groups) * n_heads * kCounterStride;
}

hipError_t launch_decode_f16(const DecodeArgs& a, hipStream_t s) {
  if (a.n_groups <= 0 || a.n_splits <= 0) return hipSuccess;
  const dim3 grid(a.n_splits, a.n_heads, a.n_groups), block(kWgThreads);
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

