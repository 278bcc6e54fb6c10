// Decode-step attention: one new query row per beam / slot against cached K/V.
//
// K2 (decode_f16): split-K attention over the f16 KV cache
//   (replaces crates/tensor/src/ops/attention.rs:246-434 single_token_mha_d64
//    as called from crates/whisper/src/decoder.rs:636 / :698).
//   Grid (split, head, group). A workgroup owns kChunk = 128 consecutive keys
//   of one (group, head) plane and ALL query rows of the group (the beams of
//   an utterance share the cross-attention plane, so it is read once per step
//   instead of once per beam). Every thread issues its q load and all its K and
//   V loads (2 keys x 2 x 16 B each) before any arithmetic, so the whole
//   layer's cache is in flight from the first cycles.
//   Partials (max, sum, acc[64]) per row are published with agent-scope
//   (sc1, L2-coherent) stores; after every wave has waited for its stores, one
//   thread bumps the (group, head) counter -- each on its own 128-byte line, so
//   the increments of different heads do not serialize. The workgroup that
//   sees the last count merges all splits with the log-sum-exp rule, reading
//   the partials with agent-scope loads (all splits at once up to 12 splits,
//   else 16 at a time), writes the output and re-arms its counter. Agent-scope atomics avoid the full-L2 writeback
//   and invalidate that a device-wide __threadfence costs on gfx950.
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
constexpr int kChunk = kDecodeChunk;  // keys per workgroup: 2 per thread, 4 threads per key
constexpr int kKpt = kChunk / 64;
constexpr int kPart = 68;    // floats per partial row: m, l, 2 pad, acc[64]
constexpr int kCounterStride = 32;  // 128 bytes between merge counters
constexpr int kMergeBatch = 16;     // partial loads in flight per thread (long rows)
constexpr int kMaxSplitsMerge = 12; // splits merged in one round (rows up to 1536 keys)

// Cross-lane moves inside a row of 16 lanes (DPP): xor 1, xor 2, mirror-8, mirror-16.
template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                0xF, 0xF, false));
}
__device__ inline float quad_sum(float x) {
  x += dpp<0xB1>(x);
  return x + dpp<0x4E>(x);
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
  const int part = tid & 3, kl0 = tid >> 2;

  // Query rows of this head first (row tid/64 and row tid/64 + 4), then every
  // cache load of the workgroup.
  const int qr = tid >> 6, qd = tid & 63;
  const float* qbase = a.q + static_cast<int64_t>(g * rows) * a.q_rs + h * 64 + qd;
  float qv0 = 0.f, qv1 = 0.f;
  if (qr < rows) qv0 = qbase[static_cast<int64_t>(qr) * a.q_rs];
  if (R > 4 && qr + 4 < rows) qv1 = qbase[static_cast<int64_t>(qr + 4) * a.q_rs];
  u32x4 kx[kKpt][2], vx[kKpt][2];
  const _Float16* kplane = a.k + a.goff[g] + h * a.kv_hs;
  const _Float16* vplane = a.v + a.goff[g] + h * a.kv_hs;
#pragma unroll
  for (int i = 0; i < kKpt; ++i) {
    const int key = split * kChunk + kl0 + 64 * i;
    if (key < len) {
      const _Float16* kp = kplane + static_cast<int64_t>(key) * 64 + part * 16;
      const _Float16* vp = vplane + static_cast<int64_t>(key) * 64 + part * 16;
      kx[i][0] = *reinterpret_cast<const u32x4*>(kp);
      kx[i][1] = *reinterpret_cast<const u32x4*>(kp + 8);
      vx[i][0] = *reinterpret_cast<const u32x4*>(vp);
      vx[i][1] = *reinterpret_cast<const u32x4*>(vp + 8);
    } else {
      kx[i][0] = kx[i][1] = vx[i][0] = vx[i][1] = u32x4{0, 0, 0, 0};
    }
  }
  if (qr < R) qs[qr][qd] = qv0 * a.scale_log2;  // rows >= `rows` hold zeros
  if (R > 4 && qr + 4 < R) qs[qr + 4][qd] = qv1 * a.scale_log2;
  __syncthreads();

  // Scores in the exp2 domain: 16-wide partial dots, summed over the 4 lanes
  // of a key with DPP.
#pragma unroll
  for (int i = 0; i < kKpt; ++i) {
    const int kl = kl0 + 64 * i;
    const bool valid = split * kChunk + kl < len;
    const f16x8 ka = __builtin_bit_cast(f16x8, kx[i][0]);
    const f16x8 kb = __builtin_bit_cast(f16x8, kx[i][1]);
    float kf[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kf[j] = static_cast<float>(ka[j]);
      kf[8 + j] = static_cast<float>(kb[j]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s = __builtin_fmaf(qs[r][part * 16 + j], kf[j], s);
      s = quad_sum(s);
      if (part == 0) ps[r][kl] = valid ? s : -INFINITY;
    }
    *reinterpret_cast<u32x4*>(&vs[kl][part * 16]) = vx[i][0];
    *reinterpret_cast<u32x4*>(&vs[kl][part * 16 + 8]) = vx[i][1];
  }
  __syncthreads();

  // Chunk softmax statistics: one wave per row.
  const int wave = tid >> 6, lane = tid & 63;
  for (int r = wave; r < R; r += 4) {
    float x[kKpt], mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kKpt; ++i) {
      x[i] = ps[r][lane + 64 * i];
      mx = fmaxf(mx, x[i]);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kKpt; ++i) {
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

  // P V over the chunk: thread (quarter, d) sums 32 keys for every row.
  {
    const int d = tid & 63, qq = tid >> 6;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll 8
    for (int i = 0; i < kChunk / 4; ++i) {
      const int kk = qq * (kChunk / 4) + i;
      const float vv = static_cast<float>(vs[kk][d]);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = __builtin_fmaf(ps[r][kk], vv, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) red[qq][r][d] = acc[r];
  }
  __syncthreads();

  if (a.n_splits == 1) {
    // The whole row in one workgroup: normalize and store directly.
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
    st_agent(mine + r * kPart + 4 + d, red[0][r][d] + red[1][r][d] + red[2][r][d] + red[3][r][d]);
  }
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

  // Log-sum-exp merge of all splits (exp2 domain).
  const float* base = a.part + static_cast<int64_t>(gh) * a.n_splits * rows * kPart;
  const int ns = a.n_splits;
  if (ns <= kMaxSplitsMerge) {
    // One round: a thread merges two (row, d) elements and issues the partial
    // loads of both, for every split, before any arithmetic.
    for (int e0 = tid; e0 < rows * 64; e0 += 2 * kThreads) {
      const int e1 = e0 + kThreads;
      const bool two = e1 < rows * 64;
      const int r0 = e0 >> 6, r1 = two ? (e1 >> 6) : r0, d0 = e0 & 63, d1 = e1 & 63;
      float m0[kMaxSplitsMerge], l0[kMaxSplitsMerge], x0[kMaxSplitsMerge];
      float m1[kMaxSplitsMerge], l1[kMaxSplitsMerge], x1[kMaxSplitsMerge];
#pragma unroll
      for (int sp = 0; sp < kMaxSplitsMerge; ++sp) {
        m0[sp] = m1[sp] = -INFINITY;
        l0[sp] = l1[sp] = x0[sp] = x1[sp] = 0.f;
        if (sp < ns) {
          const float* p0 = base + (sp * rows + r0) * kPart;
          m0[sp] = ld_agent(p0);
          l0[sp] = ld_agent(p0 + 1);
          x0[sp] = ld_agent(p0 + 4 + d0);
          if (two) {
            const float* p1 = base + (sp * rows + r1) * kPart;
            m1[sp] = ld_agent(p1);
            l1[sp] = ld_agent(p1 + 1);
            x1[sp] = ld_agent(p1 + 4 + d1);
          }
        }
      }
      float M0 = -INFINITY, M1 = -INFINITY;
#pragma unroll
      for (int sp = 0; sp < kMaxSplitsMerge; ++sp) {
        M0 = fmaxf(M0, m0[sp]);
        M1 = fmaxf(M1, m1[sp]);
      }
      float L0 = 0.f, A0 = 0.f, L1 = 0.f, A1 = 0.f;
#pragma unroll
      for (int sp = 0; sp < kMaxSplitsMerge; ++sp) {
        const float w0 = (m0[sp] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m0[sp] - M0);
        const float w1 = (m1[sp] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m1[sp] - M1);
        L0 = __builtin_fmaf(l0[sp], w0, L0);
        A0 = __builtin_fmaf(x0[sp], w0, A0);
        L1 = __builtin_fmaf(l1[sp], w1, L1);
        A1 = __builtin_fmaf(x1[sp], w1, A1);
      }
      a.o[static_cast<int64_t>(g * rows + r0) * a.o_rs + h * 64 + d0] = L0 > 0.f ? A0 * (1.f / L0) : 0.f;
      if (two)
        a.o[static_cast<int64_t>(g * rows + r1) * a.o_rs + h * 64 + d1] = L1 > 0.f ? A1 * (1.f / L1) : 0.f;
    }
  } else {
    // Longer rows: batches of kMergeBatch splits with their loads issued
    // together, folded online across batches.
    for (int e = tid; e < rows * 64; e += kThreads) {
      const int r = e >> 6, d = e & 63;
      float M = -INFINITY, L = 0.f, acc = 0.f;
      for (int s0 = 0; s0 < ns; s0 += kMergeBatch) {
        float ms[kMergeBatch], ls[kMergeBatch], as[kMergeBatch];
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
          ms[j] = -INFINITY;
          ls[j] = as[j] = 0.f;
          if (s0 + j < ns) {
            const float* pr = base + ((s0 + j) * rows + r) * kPart;
            ms[j] = ld_agent(pr);
            ls[j] = ld_agent(pr + 1);
            as[j] = ld_agent(pr + 4 + d);
          }
        }
        float Mb = M;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) Mb = fmaxf(Mb, ms[j]);
        if (Mb == -INFINITY) continue;
        const float scale = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - Mb);
        L *= scale;
        acc *= scale;
#pragma unroll
        for (int j = 0; j < kMergeBatch; ++j) {
          const float w = (ms[j] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms[j] - Mb);
          L = __builtin_fmaf(ls[j], w, L);
          acc = __builtin_fmaf(as[j], w, acc);
        }
        M = Mb;
      }
      a.o[static_cast<int64_t>(g * rows + r) * a.o_rs + h * 64 + d] = L > 0.f ? acc * (1.f / L) : 0.f;
    }
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
