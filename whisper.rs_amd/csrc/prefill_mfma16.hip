// K1: flash-attention prefill on gfx950 MFMA, d_head = 64, f16 or bf16 inputs,
// f32 softmax statistics and accumulators, f32 output.
//
// Semantics follow crates/tensor/src/ops/attention.rs:68-243 (online softmax
// over key tiles, causal mask j <= i [+ offset], fully masked rows -> 0,
// out = acc * (1/l) or 0 when l == 0). The arithmetic differs only in
// summation order and in rounding the softmax weights to f16 before the PV
// product; the row sum l is accumulated from those same rounded weights, so the
// output is an exact convex combination of V rows with the rounded weights.
//
// Work decomposition: one workgroup = 4 waves = 128 queries of one
// (window, head); each wave owns 32 queries. Per 64-key tile:
//   S^T[64 keys x 32 q] = K_tile[64 x 64] . Q^T      (2 x 4 MFMA 32x32x16)
//   O^T[64 d x 32 q]   += V_tile^T[64 x 64] . P^T    (2 x 4 MFMA 32x32x16 f16)
// Computing S^T (keys on the MFMA M axis) puts one query per lane, so the row
// max / row sum are register reductions plus a single swap with lane^32, and
// the S^T accumulator registers are, after exp2 and packing, exactly the B
// operand of the PV product (the contraction over keys is summed in the key
// order the accumulator layout hands out; V^T is read from LDS in the same
// order).
#include "wrs_internal.hpp"

namespace wrs {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 64;         // head width of every Whisper model
constexpr int kM = 128;        // queries per workgroup (32 per wave)
constexpr int kN = 64;         // keys per tile
constexpr int kThreads = 256;  // 4 waves of 64
constexpr int kKs = 72;        // LDS row pitch of the K tile, in 16-bit elements
constexpr int kVs = 72;        // LDS row pitch of the transposed V tile
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct Elem;

template <>
struct Elem<_Float16> {
  static __device__ inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ inline u32x4 to_f16(u32x4 x) { return x; }
};

template <>
struct Elem<__bf16> {
  static __device__ inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // bf16 -> f16 for the PV product: widening to f32 is a shift and the f32 ->
  // f16 rounding is exact for bf16 values inside the f16 normal range.
  static __device__ inline u32x4 to_f16(u32x4 x) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x2 w = {__builtin_bit_cast(float, x[i] << 16),
                 __builtin_bit_cast(float, x[i] & 0xffff0000u)};
      r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(w, f16x2));
    }
    return r;
  }
};

__device__ inline f32x16 mfma_f16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Logical workgroup id with an XCD-aware remap: the hardware hands linear ids
// round-robin to the 8 XCDs, so consecutive logical ids (the query blocks of
// one (window, head), which read the same K/V) are gathered onto one XCD and
// share its L2.
__device__ inline int xcd_remap(int pid, int nwg) {
  const int xcd = pid & 7, k = pid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  return xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
}

template <typename T>
__global__ __launch_bounds__(kThreads, 2) void fa2_prefill_d64(PrefillArgs a, int n_qblk) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kN * kKs];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD * kVs];

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int qblk = lid % n_qblk;
  const int bh = lid / n_qblk;
  const int h = bh % a.n_heads;
  const int b = bh / a.n_heads;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, hl = lane >> 5;

  const T* qp = static_cast<const T*>(a.q) + b * a.lq.bs + h * a.lq.hs;
  const T* kp = static_cast<const T*>(a.k) + b * a.lk.bs + h * a.lk.hs;
  const T* vp = static_cast<const T*>(a.v) + b * a.lv.bs + h * a.lv.hs;

  // This lane's query: column r32 of the wave's S^T block.
  const int qi = qblk * kM + wave * 32 + r32;
  const int qpos = qi + a.q_pos_offset;
  u32x4 qf[4];
  if (qi < a.t_q) {
    const T* row = qp + static_cast<int64_t>(qi) * a.lq.rs + hl * 8;
#pragma unroll
    for (int dk = 0; dk < 4; ++dk) qf[dk] = *reinterpret_cast<const u32x4*>(row + dk * 16);
  } else {
#pragma unroll
    for (int dk = 0; dk < 4; ++dk) qf[dk] = u32x4{0, 0, 0, 0};
  }

  int kv_end = a.t_kv;
  if (a.causal) {
    // No query of this block reaches past its last row (attention.rs:132-134).
    const int last = min(qblk * kM + kM, a.t_q) - 1 + a.q_pos_offset;
    kv_end = min(kv_end, last + 1);
  }

  const float c = a.scale * kLog2e;  // exp(scale*s - m') == exp2(c*s - c*m)
  f32x16 o0 = {}, o1 = {};           // O^T rows d 0..31 and 32..63, column = query
  float m = -INFINITY;               // running max of raw q.k for this query
  float l = 0.f;                     // running sum over this lane's key half

  for (int j0 = 0; j0 < kv_end; j0 += kN) {
    __syncthreads();
    // K tile -> LDS, row-major [key][d]; keys past t_kv are zero.
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int ci = tid + r * kThreads;
      const int key = ci >> 3, dp = ci & 7;
      u32x4 val = {0, 0, 0, 0};
      if (j0 + key < a.t_kv)
        val = *reinterpret_cast<const u32x4*>(kp + static_cast<int64_t>(j0 + key) * a.lk.rs +
                                              dp * 8);
      *reinterpret_cast<u32x4*>(Ks + key * kKs + dp * 8) = val;
    }
    // V tile -> LDS transposed [d][key] as f16, two keys packed per dword.
    {
      const int pr = tid >> 3, dp = tid & 7;
      const int key = j0 + 2 * pr;
      u32x4 x0 = {0, 0, 0, 0}, x1 = {0, 0, 0, 0};
      if (key < a.t_kv)
        x0 = *reinterpret_cast<const u32x4*>(vp + static_cast<int64_t>(key) * a.lv.rs + dp * 8);
      if (key + 1 < a.t_kv)
        x1 = *reinterpret_cast<const u32x4*>(vp + static_cast<int64_t>(key + 1) * a.lv.rs +
                                             dp * 8);
      x0 = Elem<T>::to_f16(x0);
      x1 = Elem<T>::to_f16(x1);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = (x0[w] & 0xffffu) | (x1[w] << 16);
        const uint32_t hi = (x0[w] >> 16) | (x1[w] & 0xffff0000u);
        *reinterpret_cast<uint32_t*>(Vt + (dp * 8 + 2 * w) * kVs + 2 * pr) = lo;
        *reinterpret_cast<uint32_t*>(Vt + (dp * 8 + 2 * w + 1) * kVs + 2 * pr) = hi;
      }
    }
    __syncthreads();

    // S^T = K Q^T for keys [j0, j0+32) and [j0+32, j0+64).
    f32x16 s0 = {}, s1 = {};
#pragma unroll
    for (int dk = 0; dk < 4; ++dk) {
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(Ks + r32 * kKs + dk * 16 + hl * 8);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(Ks + (32 + r32) * kKs + dk * 16 + hl * 8);
      s0 = Elem<T>::mfma(a0, qf[dk], s0);
      s1 = Elem<T>::mfma(a1, qf[dk], s1);
    }

    // Accumulator register i of a 32x32 block holds row 8*(i/4) + 4*hl + i%4.
    const bool need_mask = a.causal || (j0 + kN > a.t_kv);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (need_mask) {
        const int kr = j0 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (kr >= a.t_kv || (a.causal && kr > qpos)) s0[i] = -INFINITY;
        if (kr + 32 >= a.t_kv || (a.causal && kr + 32 > qpos)) s1[i] = -INFINITY;
      }
      mx = fmaxf(mx, fmaxf(s0[i], s1[i]));
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m - m_use) * c);
    const float mc = m_use * c;
    m = m_new;

    // P^T in f16, already in B-operand order: PV block kb2 covers tile keys
    // 16*kb2 + 8*(j/4) + 4*hl + j%4 for element j.
    u32x4 pb[4];
    float ls = 0.f;
#pragma unroll
    for (int kb2 = 0; kb2 < 4; ++kb2) {
      const int base = 8 * (kb2 & 1);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float x0 = (kb2 < 2) ? s0[base + 2 * w] : s1[base + 2 * w];
        const float x1 = (kb2 < 2) ? s0[base + 2 * w + 1] : s1[base + 2 * w + 1];
        const f32x2 pp = {__builtin_amdgcn_exp2f(__builtin_fmaf(x0, c, -mc)),
                          __builtin_amdgcn_exp2f(__builtin_fmaf(x1, c, -mc))};
        const f16x2 hp = __builtin_convertvector(pp, f16x2);
        ls = __builtin_amdgcn_fdot2(hp, f16x2{1.0f16, 1.0f16}, ls, false);
        pb[kb2][w] = __builtin_bit_cast(uint32_t, hp);
      }
    }
    l = l * alpha + ls;
    o0 *= alpha;
    o1 *= alpha;

#pragma unroll
    for (int kb2 = 0; kb2 < 4; ++kb2) {
      const uint16_t* v0 = Vt + r32 * kVs + 16 * kb2 + 4 * hl;
      const uint16_t* v1 = v0 + 32 * kVs;
      const u32x2 a0l = *reinterpret_cast<const u32x2*>(v0);
      const u32x2 a0h = *reinterpret_cast<const u32x2*>(v0 + 8);
      const u32x2 a1l = *reinterpret_cast<const u32x2*>(v1);
      const u32x2 a1h = *reinterpret_cast<const u32x2*>(v1 + 8);
      o0 = mfma_f16(u32x4{a0l.x, a0l.y, a0h.x, a0h.y}, pb[kb2], o0);
      o1 = mfma_f16(u32x4{a1l.x, a1l.y, a1h.x, a1h.y}, pb[kb2], o1);
    }
  }

  l += __shfl_xor(l, 32);
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
  if (qi < a.t_q) {
    float* op = a.o + b * a.lo.bs + h * a.lo.hs + static_cast<int64_t>(qi) * a.lo.rs;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *reinterpret_cast<f32x4*>(op + 8 * g + 4 * hl) =
          f32x4{o0[4 * g], o0[4 * g + 1], o0[4 * g + 2], o0[4 * g + 3]} * inv;
      *reinterpret_cast<f32x4*>(op + 32 + 8 * g + 4 * hl) =
          f32x4{o1[4 * g], o1[4 * g + 1], o1[4 * g + 2], o1[4 * g + 3]} * inv;
    }
  }
}

}  // namespace

hipError_t launch_prefill_mfma16(const PrefillArgs& a, DType dt, hipStream_t s) {
  const int n_qblk = (a.t_q + kM - 1) / kM;
  const int64_t nwg = static_cast<int64_t>(n_qblk) * a.n_heads * a.batch;
  if (nwg <= 0) return hipSuccess;
  if (nwg > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nwg)), block(kThreads);
  if (dt == kF16)
    hipLaunchKernelGGL(fa2_prefill_d64<_Float16>, grid, block, 0, s, a, n_qblk);
  else
    hipLaunchKernelGGL(fa2_prefill_d64<__bf16>, grid, block, 0, s, a, n_qblk);
  return hipGetLastError();
}

}  // namespace wrs
