// K4: flash-attention prefill with f32 operands on gfx950 f32 MFMA
// (v_mfma_f32_32x32x2_f32), for the 1e-5 accumulate-check runs and for the
// shapes the 16-bit kernel does not take (d_head != 64, f32 queries against
// the f16 decoder cache). One workgroup runs one 128-query block
// (prefill_f32_block.hpp holds the block routine and its semantics).
#include "prefill_f32_block.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace wrs {
namespace {

using f32blk::fa2_block;
using f32blk::kM;
using f32blk::kThreads;
using f32blk::Tiles;
using f32blk::f32x16;


template <typename QT, typename KT, int DB>
__global__ __launch_bounds__(kThreads, 1) void fa2_prefill_f32(PrefillArgs a, int n_qblk) {
  __shared__ Tiles<DB> tl;
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = lid / n_qblk;
  fa2_block<QT, KT, DB, 4, true>(a, (lid % n_qblk) * f32blk::kM, bh % a.n_heads, bh / a.n_heads, tl);
}

// Small grids of 128-query blocks (whisper-tiny's encoder: 12 blocks x 6
// heads = 72) leave most SIMDs idle, since one wave carries 32 queries through
// every key. fa2_prefill_f32_ksplit runs one 32-query block per workgroup
// instead, with S = 4 waves (2..4 when forced) that take the block's key tiles
// in turn (tile t on wave t % S). Each wave keeps its own online softmax over
// its tiles, in its own LDS tile pair, with the next tile's rows loading while
// it computes. The workgroup then merges the S (max, sum, O) by the
// log-sum-exp rule. Grids of fewer such blocks than half the CUs (a 64-query
// cross-attention call: 12 blocks for 6 heads) spread each block over `ws`
// workgroups, wave w of workgroup s taking the block's tiles s S + w,
// s S + w + S ws, ...; each workgroup publishes its merged (max, sum, O) rows
// with agent-scope stores, and the last of the block's workgroups to count in
// folds them in split order (bits independent of arrival order), re-arms the
// block's counter and writes the rows.
// exp(x) as the hardware's exp2 of x log2(e). For the softmax's x <= 0 the
// rounding of the product moves a weight e^x by at most |x| e^x 2^-24, below
// 2.2e-8 absolute; libm's expf is a ~10-instruction range reduction.
__device__ inline float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f); }

constexpr int kQS = 32;       // queries per k-split workgroup
constexpr int kMaxSplit = 4;  // waves per k-split workgroup, at most
constexpr int kMaxWs = 16;    // workgroups per block, at most
constexpr int kWsCounterStride = 32;  // words between merge counters (one 128-byte line)

template <typename QT, typename KT, int DB>
__global__ __launch_bounds__(64 * kMaxSplit, DB <= 2 ? 2 : 1) void fa2_prefill_f32_ksplit(
    PrefillArgs a, int n_qblk, int vec, int ws) {
  constexpr int D = 32 * DB;
  constexpr int P = Tiles<DB>::P;
  constexpr int kN = f32blk::kN;
  constexpr int R = D + 1;  // merge row pitch: the 32 queries of one write hit distinct banks
  __shared__ Tiles<DB> tl[kMaxSplit];
  static_assert(sizeof(Tiles<DB>) >= (kQS * R + 2 * kQS) * sizeof(float), "merge rows fit");
  typedef float f32x4 __attribute__((ext_vector_type(4)));

  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  // A block's ws workgroups are neighbours in lid (one XCD).
  const int wsplit = lid % ws, blk = lid / ws;
  const int qblk = blk % n_qblk;
  const int bh = blk / n_qblk;
  const int h = bh % a.n_heads, b = bh / a.n_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = __builtin_amdgcn_readfirstlane(static_cast<int>(blockDim.x) >> 6);
  // This wave's first tile and the stride between its tiles.
  const int j_first = (wsplit * S + wave) * kN, j_step = S * ws * kN;
  const int r32 = lane & 31, hl = lane >> 5;
  const int dh = a.d_head;
  float* const Ks = tl[wave].k;
  float* const Vs = tl[wave].v;

  const QT* qp = static_cast<const QT*>(a.q) + b * a.lq.bs + h * a.lq.hs;
  const KT* kp = static_cast<const KT*>(a.k) + b * a.lk.bs + h * a.lk.hs;
  const KT* vp = static_cast<const KT*>(a.v) + b * a.lv.bs + h * a.lv.hs;

  const int qi = qblk * kQS + r32;
  const int qpos = qi + a.q_pos_offset;
  const int nth = 64 * S;
  // The block's 32 query rows go through LDS (wave 0's K tile, pitch P) in
  // coalesced loads shared by the S waves; each lane then takes its 32-row
  // MFMA operand (d = 2 kk + hl) from there. Loads past the block's rows or
  // d_head read row 0 of the head and are stored as 0.
  float qf[D / 2];
  auto stage_q = [&] {
    float* const qs = tl[0].k;
    for (int e0 = 0; e0 < kQS * D; e0 += 8 * nth) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + u * nth + tid, mq = e / D, d = e % D;
        const bool ok = e < kQS * D && qblk * kQS + mq < a.t_q && d < dh;
        x[u] = f32blk::widen(qp[ok ? static_cast<int64_t>(qblk * kQS + mq) * a.lq.rs + d : 0]);
        x[u] = ok ? x[u] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + u * nth + tid;
        if (e < kQS * D) qs[(e / D) * P + e % D] = x[u];
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < D / 2; ++kk) qf[kk] = qs[r32 * P + 2 * kk + hl];
    __syncthreads();  // the tile loop reuses the buffer
  };
  int kv_end = a.t_kv;
  if (a.causal) {
    const int last = min(qblk * kQS + kQS, a.t_q) - 1 + a.q_pos_offset;
    kv_end = min(kv_end, last + 1);
  }

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x16{};
  float m = -INFINITY, l = 0.f;

  auto wave_sync = [] {
    // LDS operations of one wave complete in order: this orders the wave's
    // tile reads before its next writes, and its writes before its reads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // The same per-tile arithmetic as fa2_block (attention.rs:141-222).
  auto tile = [&](int j0) {
    // Two independent accumulator chains over d: with one wave per SIMD a
    // single chain would wait out every MFMA's latency.
    f32x16 sp[2] = {};
#pragma unroll
    for (int kk = 0; kk < D / 2; ++kk)
      sp[kk & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[r32 * P + 2 * kk + hl], qf[kk],
                                                         sp[kk & 1], 0, 0, 0);
    f32x16 sc = sp[0] + sp[1];
    // Tiles wholly inside the key range (and, with the causal mask, at or
    // below the block's first query position) need no masking.
    const bool whole = j0 + kN <= a.t_kv && (!a.causal || j0 + kN - 1 <= qblk * kQS + a.q_pos_offset);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float x = a.scale * sc[i];
      if (!whole) {
        const int key = j0 + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (key >= a.t_kv || (a.causal && key > qpos)) x = -INFINITY;
      }
      sc[i] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float alpha = (m == -INFINITY) ? 0.f : fexp(m - m_new);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    m = m_new;
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sc[i] = fexp(sc[i] - m_use);
      ls += sc[i];
    }
    l = l * alpha + ls;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= alpha;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int key = 8 * (t >> 2) + 4 * hl + (t & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[key * P + db * 32 + r32], sc[t], o[db],
                                                     0, 0, 0);
    }
  };

  if constexpr (std::is_same<KT, float>::value) {
    if (vec) {
      // f32 K/V rows of exactly D floats, 16-byte aligned: float4 f = lane +
      // 64 i of the tile (key f / (D/4), column 4 (f % (D/4))), so each load
      // instruction covers whole rows; one tile ahead of the tile computed.
      // Keys past t_kv read the last key and are stored as 0.
      constexpr int C4 = D / 4;
      f32x4 kr[D / 8], vr[D / 8];
      auto load = [&](int j0) {
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
          const int f = lane + 64 * i, key = j0 + f / C4, c = 4 * (f % C4);
          const int64_t row = min(key, a.t_kv - 1);
          kr[i] = *reinterpret_cast<const f32x4*>(kp + row * a.lk.rs + c);
          vr[i] = *reinterpret_cast<const f32x4*>(vp + row * a.lv.rs + c);
          if (key >= a.t_kv) kr[i] = vr[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      };
      int j0 = j_first;
      if (j0 < kv_end) load(j0);
      stage_q();
      for (; j0 < kv_end; j0 += j_step) {
        wave_sync();
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
          const int f = lane + 64 * i, at = (f / C4) * P + 4 * (f % C4);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            Ks[at + c] = kr[i][c];
            Vs[at + c] = vr[i][c];
          }
        }
        wave_sync();
        if (j0 + j_step < kv_end) load(j0 + j_step);
        tile(j0);
      }
    }
  }
  if (!(std::is_same<KT, float>::value && vec)) {
    stage_q();
    for (int j0 = j_first; j0 < kv_end; j0 += j_step) {
      wave_sync();
#pragma unroll 4
      for (int e = lane; e < kN * D; e += 64) {
        const int key = e / D, d = e % D;
        float kv = 0.f, vv = 0.f;
        if (j0 + key < a.t_kv && d < dh) {
          kv = f32blk::widen(kp[static_cast<int64_t>(j0 + key) * a.lk.rs + d]);
          vv = f32blk::widen(vp[static_cast<int64_t>(j0 + key) * a.lv.rs + d]);
        }
        Ks[key * P + d] = kv;
        Vs[key * P + d] = vv;
      }
      wave_sync();
      tile(j0);
    }
  }
  l += __shfl_xor(l, 32);

  // Merge rows in the wave's own tile pair (both tiles, as one array): O
  // [32][R] (query-major), then m and l per query.
  __syncthreads();  // every wave is past its last tile reads
  float* const mo = reinterpret_cast<float*>(&tl[wave]);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = db * 32 + 8 * (i >> 2) + 4 * hl + (i & 3);
      mo[r32 * R + d] = o[db][i];
    }
  if (hl == 0) {
    mo[kQS * R + r32] = m;
    mo[kQS * R + kQS + r32] = l;
  }
  __syncthreads();
  // Per query row: the waves' weights e_w = exp(m_w - M) (0 for an empty
  // wave) and the total sum L = sum_w e_w l_w, in wave order.
  __shared__ float wts[kMaxSplit + 1][kQS];
  auto mrow = [&](int w) { return reinterpret_cast<const float*>(&tl[w]); };
  if (tid < kQS) {
    float mw[kMaxSplit], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMaxSplit; ++w) {
      mw[w] = w < S ? mrow(w)[kQS * R + tid] : -INFINITY;
      M = fmaxf(M, mw[w]);
    }
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < kMaxSplit; ++w) {
      const float ew = (mw[w] == -INFINITY) ? 0.f : expf(mw[w] - M);
      wts[w][tid] = ew;
      if (w < S) L += ew * mrow(w)[kQS * R + kQS + tid];
    }
    wts[kMaxSplit][tid] = L;
    if (ws > 1) {
      // Published rows: [max, sum, O...], dh + 2 floats per (block, split).
      float* const mine = a.split_part + (static_cast<int64_t>(blk) * ws + wsplit) * kQS * (dh + 2);
      st_agent(mine + tid * (dh + 2), M);
      st_agent(mine + tid * (dh + 2) + 1, L);
    }
  }
  __syncthreads();
  // Output element e = (row e / dh, column e % dh): sum_w e_w O_w, eight
  // elements per thread at a time with all their LDS reads in flight. With
  // ws == 1 it is normalized and stored; otherwise published unnormalized.
  const int pitch = dh + 2;
  float* const mine = a.split_part + (static_cast<int64_t>(blk) * ws + wsplit) * kQS * pitch;
  const int ne = kQS * dh;
  for (int e0 = 0; e0 < ne; e0 += 8 * nth) {
    float acc[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = min(e0 + u * nth + tid, ne - 1), mq = e / dh, d = e % dh;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kMaxSplit; ++w)
        if (w < S) sum += wts[w][mq] * mrow(w)[mq * R + d];
      acc[u] = sum;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + u * nth + tid, mq = e / dh, d = e % dh;
      const int oq = qblk * kQS + mq;
      if (e >= ne || oq >= a.t_q) continue;
      if (ws == 1) {
        const float L = wts[kMaxSplit][mq];
        a.o[b * a.lo.bs + h * a.lo.hs + static_cast<int64_t>(oq) * a.lo.rs + d] =
            acc[u] * ((L > 0.f) ? 1.f / L : 0.f);
      } else {
        st_agent(mine + mq * pitch + 2 + d, acc[u]);
      }
    }
  }
  if (ws == 1) return;
  __shared__ int merger;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  unsigned* const counter = a.split_counters + static_cast<int64_t>(blk) * kWsCounterStride;
  if (tid == 0)
    merger = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             static_cast<unsigned>(ws - 1);
  __syncthreads();
  if (!merger) return;
  // The fold, in split order (bits independent of arrival order): the rows'
  // max and sum of every split into LDS (the tile buffers are free), then per
  // row the weight of each split and the total sum, then each output element
  // from its splits' partial sums. Every round of loads is unrolled and
  // unconditional (clamped indices), so all of a round is in flight at once.
  const float* const all = a.split_part + static_cast<int64_t>(blk) * ws * kQS * pitch;
  float* const sm = reinterpret_cast<float*>(&tl[0]);  // [kMaxWs][kQS] max, then weight
  float* const sl = sm + kMaxWs * kQS;                 // [kMaxWs][kQS] sum
  float* const sinv = sl + kMaxWs * kQS;               // [kQS] 1 / total sum, or 0
  static_assert(sizeof(Tiles<DB>) >= (2 * kMaxWs + 1) * kQS * sizeof(float), "fold fits");
  // The first round carries the statistics and the first kF elements per
  // thread; the barriers around the weights wait on LDS only, so those
  // elements' loads stay in flight through them.
  constexpr int kF = 8;
  auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  float part[kF][kMaxWs];
  // With d_head even, element pairs (d, d + 1) of a row are one 8-byte
  // agent-scope load: a thread's kF elements are kF / 2 pairs.
  const bool pairs = (dh & 1) == 0;
  auto elem = [&](int e0, int u) {
    return pairs ? e0 + 2 * ((u >> 1) * nth + tid) + (u & 1) : e0 + u * nth + tid;
  };
  auto fold_load = [&](int e0) {
    if (pairs) {
#pragma unroll
      for (int u = 0; u < kF; u += 2) {
        const int e = min(elem(e0, u), ne - 2), mq = e / dh, d = e % dh;
#pragma unroll
        for (int s2 = 0; s2 < kMaxWs; ++s2) {
          const unsigned long long w = __hip_atomic_load(
              reinterpret_cast<const unsigned long long*>(all + ((s2 < ws ? s2 : 0) * kQS + mq) * pitch + 2 + d),
              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          part[u][s2] = __uint_as_float(static_cast<unsigned>(w));
          part[u + 1][s2] = __uint_as_float(static_cast<unsigned>(w >> 32));
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kF; ++u) {
        const int e = min(elem(e0, u), ne - 1), mq = e / dh, d = e % dh;
#pragma unroll
        for (int s2 = 0; s2 < kMaxWs; ++s2)
          part[u][s2] = ld_agent(all + ((s2 < ws ? s2 : 0) * kQS + mq) * pitch + 2 + d);
      }
    }
  };
  auto fold_store = [&](int e0) {
#pragma unroll
    for (int u = 0; u < kF; ++u) {
      const int e = elem(e0, u), mq = e / dh, d = e % dh;
      const int oq = qblk * kQS + mq;
      if (e >= ne || oq >= a.t_q) continue;
      float acc = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < kMaxWs; ++s2)
        if (s2 < ws) acc += sm[s2 * kQS + mq] * part[u][s2];
      a.o[b * a.lo.bs + h * a.lo.hs + static_cast<int64_t>(oq) * a.lo.rs + d] = acc * sinv[mq];
    }
  };
  {
    constexpr int kU = kMaxWs * kQS / 128;  // nth >= 128
    const int nst = ws * kQS;
    float mx[kU], lx[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const float* const r = all + min(u * nth + tid, nst - 1) * pitch;  // split i / kQS, row i % kQS
      mx[u] = ld_agent(r);
      lx[u] = ld_agent(r + 1);
    }
    fold_load(0);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = u * nth + tid;
      if (i < nst) {
        sm[i] = mx[u];
        sl[i] = lx[u];
      }
    }
  }
  lds_barrier();
  if (tid < kQS) {
    float ms[kMaxWs], M = -INFINITY;
#pragma unroll
    for (int s2 = 0; s2 < kMaxWs; ++s2) {
      ms[s2] = s2 < ws ? sm[s2 * kQS + tid] : -INFINITY;
      M = fmaxf(M, ms[s2]);
    }
    float L = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < kMaxWs; ++s2) {
      const float es = (ms[s2] == -INFINITY) ? 0.f : expf(ms[s2] - M);
      if (s2 < ws) {
        sm[s2 * kQS + tid] = es;
        L += es * sl[s2 * kQS + tid];
      }
    }
    sinv[tid] = (L > 0.f) ? 1.f / L : 0.f;
  }
  lds_barrier();
  fold_store(0);
  for (int e0 = kF * nth; e0 < ne; e0 += kF * nth) {
    fold_load(e0);
    fold_store(e0);
  }
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// CUs of the current device, read once.
int device_cus() {
  static const int cus = [] {
    int dev = 0, n = 256;
    if (hipGetDevice(&dev) == hipSuccess)
      (void)hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    return n;
  }();
  return cus;
}

// Waves per key-split workgroup: a.force_f32_split 2..4 forces that many.
int ksplit_waves(const PrefillArgs& a) {
  return a.force_f32_split >= 2 && a.force_f32_split <= 4 ? a.force_f32_split : kMaxSplit;
}

// Workgroups per 32-query block of the key split: by default, where the
// blocks occupy fewer than half the CUs and one workgroup would give each
// wave three tiles or more, as many as give every wave one of the block's
// 32-key tiles (at most kMaxWs, at most the CUs per block); forced
// (a.force_f32_split == 5) at least two. 1: no split.
int ksplit_ways(const PrefillArgs& a, int64_t nws, int64_t cus) {
  const int forced = a.force_f32_split;
  if (forced != 5 && (forced != -1 || 2 * nws >= cus)) return 1;
  const int64_t tiles = (a.t_kv + f32blk::kN - 1) / f32blk::kN;
  const int split = ksplit_waves(a);
  // Under three tiles per wave the fold costs more than the split saves
  // (64 queries x 6 heads over 188 keys: 18.5 against 16.4 us).
  if (forced != 5 && tiles < 3 * split) return 1;
  int64_t ws = std::min<int64_t>({kMaxWs, cus / std::max<int64_t>(nws, 1),
                                  std::max<int64_t>(1, (tiles + split - 1) / split)});
  if (forced == 5) ws = std::max<int64_t>(ws, 2);
  return static_cast<int>(ws);
}

int64_t ksplit_floats(const PrefillArgs& a, int64_t nws, int ws) {
  return nws * ws * kQS * (a.d_head + 2);
}
int64_t ksplit_words(int64_t nws) { return nws * kWsCounterStride; }

int64_t blocks32(const PrefillArgs& a) {
  return ((a.t_q + kQS - 1) / kQS) * static_cast<int64_t>(a.n_heads) * a.batch;
}

template <typename QT, typename KT>
hipError_t launch_typed(const PrefillArgs& a, hipStream_t s) {
  const int n_qblk = (a.t_q + kM - 1) / kM;
  const int64_t bh = static_cast<int64_t>(a.n_heads) * a.batch;
  const int64_t nwg = n_qblk * bh;
  if (nwg <= 0) return hipSuccess;
  const int db = (a.d_head + 31) / 32;
  if (db < 1 || db > 4) return hipErrorInvalidValue;
  // a.force_f32_split: 0 forces 128-query blocks, 1 the key split, 2..4 the
  // key split over that many waves, 5 the key split over several workgroups.
  const int forced = a.force_f32_split;
  // The key split, four waves per 32-query block, at every grid size.
  // Measured against the 128-query blocks (f32, d_head 64, 1500 queries and
  // keys): 6 heads 75 against 168 us, 32 heads 213 against 278 us, 128 heads
  // 790 against 797 us, 320 heads 1935 against 1972 us.
  const int n_qs = (a.t_q + kQS - 1) / kQS;
  const int64_t nws = n_qs * bh;
  const int split = ksplit_waves(a);
  if (forced != 0) {
    int ws = ksplit_ways(a, nws, device_cus());
    if (ws > 1 && !(a.split_part && a.split_counters &&
                    ksplit_floats(a, nws, ws) <= static_cast<int64_t>(a.split_part_floats) &&
                    ksplit_words(nws) <= static_cast<int64_t>(a.split_counter_words))) {
      // No scratch (a call under stream capture before any outside it).
      if (forced == 5) return hipErrorInvalidValue;
      ws = 1;
    }
    if (nws * ws > 0x7fffffff) return hipErrorInvalidConfiguration;
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const int vec = a.d_head == 32 * db && a.lk.rs % 4 == 0 && a.lv.rs % 4 == 0 &&
                    a.lk.bs % 4 == 0 && a.lv.bs % 4 == 0 && a.lk.hs % 4 == 0 &&
                    a.lv.hs % 4 == 0 && al16(a.k) && al16(a.v);
    const dim3 grid(static_cast<unsigned>(nws * ws)), block(64 * split);
    switch (db) {
      case 1: hipLaunchKernelGGL((fa2_prefill_f32_ksplit<QT, KT, 1>), grid, block, 0, s, a, n_qs, vec, ws); break;
      case 2: hipLaunchKernelGGL((fa2_prefill_f32_ksplit<QT, KT, 2>), grid, block, 0, s, a, n_qs, vec, ws); break;
      case 3: hipLaunchKernelGGL((fa2_prefill_f32_ksplit<QT, KT, 3>), grid, block, 0, s, a, n_qs, vec, ws); break;
      default: hipLaunchKernelGGL((fa2_prefill_f32_ksplit<QT, KT, 4>), grid, block, 0, s, a, n_qs, vec, ws); break;
    }
    return hipGetLastError();
  }
  if (nwg > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nwg)), block(kThreads);
  switch (db) {
    case 1: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 1>), grid, block, 0, s, a, n_qblk); break;
    case 2: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 2>), grid, block, 0, s, a, n_qblk); break;
    case 3: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 3>), grid, block, 0, s, a, n_qblk); break;
    default: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 4>), grid, block, 0, s, a, n_qblk); break;
  }
  return hipGetLastError();
}

}  // namespace

void prefill_f32_scratch(const PrefillArgs& a, size_t* part_floats, size_t* counter_words) {
  *part_floats = *counter_words = 0;
  const int64_t nws = blocks32(a);
  if (a.t_q <= 0 || nws <= 0 || a.force_f32_split == 0) return;
  const int ws = ksplit_ways(a, nws, device_cus());
  if (ws == 1) return;
  *part_floats = static_cast<size_t>(ksplit_floats(a, nws, ws));
  *counter_words = static_cast<size_t>(ksplit_words(nws));
}

hipError_t launch_prefill_f32(const PrefillArgs& a, DType q_dt, DType kv_dt, hipStream_t s) {
  if (q_dt == kF32 && kv_dt == kF32) return launch_typed<float, float>(a, s);
  if (q_dt == kF32 && kv_dt == kF16) return launch_typed<float, _Float16>(a, s);
  if (q_dt == kF16 && kv_dt == kF16) return launch_typed<_Float16, _Float16>(a, s);
  if (q_dt == kBF16 && kv_dt == kBF16) return launch_typed<__bf16, __bf16>(a, s);
  if (q_dt == kF32 && kv_dt == kBF16) return launch_typed<float, __bf16>(a, s);
  return hipErrorInvalidValue;
}

}  // namespace wrs
