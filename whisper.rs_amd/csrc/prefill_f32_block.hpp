// One 128-query block of the f32-operand flash-attention prefill (K4), as a
// device routine: the f32 kernel runs one per workgroup, and the bf16 16-bit
// kernel runs it for its own query rows when they came out non-finite.
//
// Semantics are those of crates/tensor/src/ops/attention.rs:68-243, step by
// step: s = scale * (q.k) (:141-156, alpha applied after the dot product),
// per-tile m_new = max(m, max_j s_j), alpha = 0 if m == -inf else
// exp(m - m_new) (:179-183), p = exp(s - m_new), l = l*alpha + sum p,
// acc = acc*alpha + P V, out = acc * (1/l) or 0 (:228-241). Only the
// summation order of the two products differs (MFMA instead of sgemm). K/V
// given as f16/bf16 are widened exactly to f32.
//
// Decomposition: 4 waves x 32 queries per 256-thread workgroup, 32-key tiles;
// the wave computes S^T = K Q^T on f32 MFMA (v_mfma_f32_32x32x2_f32) so each
// lane owns one query and its softmax statistics.
#pragma once

#include "wrs_internal.hpp"

namespace wrs {
namespace f32blk {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kM = 128;
constexpr int kN = 32;
constexpr int kThreads = 256;

template <typename T>
__device__ inline float widen(T x) {
  return static_cast<float>(x);
}

template <int DB>
struct Tiles {
  static constexpr int P = 32 * DB + 1;  // odd LDS pitch: the 32 rows of one read hit distinct banks
  float k[kN * P];
  float v[kN * P];
};

// One block of query rows: [q_begin, q_begin + 32*NW) of head h of batch
// entry b, run by NW waves (4 in the f32 kernel: a 128-query block), rows at
// or past a.t_q left alone. DB: number of 32-wide blocks covering d_head
// (<= 32*DB).
// kFast (the f32 kernel's 128-query blocks): the next tile's rows load into
// registers during the current tile, score chains over d are two, exp is the
// hardware exp2 of x log2(e), and tiles wholly inside the key range skip the
// mask. K1's bf16 recompute keeps the plain form.
template <typename QT, typename KT, int DB, int NW = 4, bool kFast = false>
__device__ inline void fa2_block(const PrefillArgs& a, int q_begin, int h, int b, Tiles<DB>& tl) {
  constexpr int D = 32 * DB;
  constexpr int P = Tiles<DB>::P;
  float* Ks = tl.k;
  float* Vs = tl.v;
  const int dh = a.d_head;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, hl = lane >> 5;

  const QT* qp = static_cast<const QT*>(a.q) + b * a.lq.bs + h * a.lq.hs;
  const KT* kp = static_cast<const KT*>(a.k) + b * a.lk.bs + h * a.lk.hs;
  const KT* vp = static_cast<const KT*>(a.v) + b * a.lv.bs + h * a.lv.hs;

  const int qi = q_begin + wave * 32 + r32;
  const int qpos = qi + a.q_pos_offset;
  // B operand of step kk: Q[qi][2*kk + hl].
  float qf[D / 2];
#pragma unroll
  for (int kk = 0; kk < D / 2; ++kk) {
    const int d = 2 * kk + hl;
    qf[kk] = (qi < a.t_q && d < dh) ? widen(qp[static_cast<int64_t>(qi) * a.lq.rs + d]) : 0.f;
  }

  int kv_end = a.t_kv;
  if (a.causal) {
    const int last = min(q_begin + 32 * NW, a.t_q) - 1 + a.q_pos_offset;
    kv_end = min(kv_end, last + 1);
  }

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x16{};
  float m = -INFINITY, l = 0.f;

  // kFast: thread tid holds elements tid + 64 NW u of the next tile.
  constexpr int kE = (kN * D + 64 * NW - 1) / (64 * NW);
  float kr[kFast ? kE : 1], vr[kFast ? kE : 1];
  auto load = [&](int j0) {
#pragma unroll
    for (int u = 0; u < kE; ++u) {
      const int e = tid + 64 * NW * u, key = e / D, d = e % D;
      const bool ok = e < kN * D && j0 + key < a.t_kv && d < dh;
      const int64_t row = min(j0 + key, a.t_kv - 1);
      const int col = min(d, dh - 1);
      kr[u] = widen(kp[row * a.lk.rs + col]);
      vr[u] = widen(vp[row * a.lv.rs + col]);
      if (!ok) kr[u] = vr[u] = 0.f;
    }
  };
  if constexpr (kFast) {
    if (kv_end > 0) load(0);
  }
  auto ex = [](float x) {
    if constexpr (kFast)
      return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f);
    else
      return expf(x);
  };

  for (int j0 = 0; j0 < kv_end; j0 += kN) {
    __syncthreads();
    if constexpr (kFast) {
#pragma unroll
      for (int u = 0; u < kE; ++u) {
        const int e = tid + 64 * NW * u;
        if (e < kN * D) {
          Ks[(e / D) * P + e % D] = kr[u];
          Vs[(e / D) * P + e % D] = vr[u];
        }
      }
      __syncthreads();
      if (j0 + kN < kv_end) load(j0 + kN);
    } else {
      for (int e = tid; e < kN * D; e += 64 * NW) {
        const int key = e / D, d = e % D;
        float kv = 0.f, vv = 0.f;
        if (j0 + key < a.t_kv && d < dh) {
          kv = widen(kp[static_cast<int64_t>(j0 + key) * a.lk.rs + d]);
          vv = widen(vp[static_cast<int64_t>(j0 + key) * a.lv.rs + d]);
        }
        Ks[key * P + d] = kv;
        Vs[key * P + d] = vv;
      }
      __syncthreads();
    }

    f32x16 s = {};
    if constexpr (kFast) {
      f32x16 s1 = {};
#pragma unroll
      for (int kk = 0; kk < D / 2; kk += 2) {
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[r32 * P + 2 * kk + hl], qf[kk], s, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[r32 * P + 2 * kk + 2 + hl], qf[kk + 1], s1,
                                                  0, 0, 0);
      }
      s += s1;
    } else {
#pragma unroll
      for (int kk = 0; kk < D / 2; ++kk)
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[r32 * P + 2 * kk + hl], qf[kk], s, 0, 0, 0);
    }

    // Tiles wholly inside the key range (and, with the causal mask, at or
    // below the block's first query position) need no masking.
    const bool whole = kFast && j0 + kN <= a.t_kv &&
                       (!a.causal || j0 + kN - 1 <= q_begin + a.q_pos_offset);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float x = a.scale * s[i];
      if (!whole) {
        const int key = j0 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (key >= a.t_kv || (a.causal && key > qpos)) x = -INFINITY;
      }
      s[i] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float alpha = (m == -INFINITY) ? 0.f : ex(m - m_new);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    m = m_new;
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = ex(s[i] - m_use);
      ls += s[i];
    }
    l = l * alpha + ls;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= alpha;

    // O^T += V^T P^T; step t contracts tile key 8*(t/4) + 4*hl + t%4, which is
    // the key this lane's accumulator register t holds.
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int key = 8 * (t >> 2) + 4 * hl + (t & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[key * P + db * 32 + r32], s[t], o[db],
                                                     0, 0, 0);
    }
  }

  l += __shfl_xor(l, 32);
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
  if (qi < a.t_q) {
    float* op = a.o + b * a.lo.bs + h * a.lo.hs + static_cast<int64_t>(qi) * a.lo.rs;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = db * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (d < dh) op[d] = o[db][i] * inv;
      }
  }
}

}  // namespace f32blk
}  // namespace wrs
