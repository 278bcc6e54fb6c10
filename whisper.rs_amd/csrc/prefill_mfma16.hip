// K1: flash-attention prefill on gfx950 MFMA, d_head = 64, f16 or bf16 inputs,
// f32 softmax statistics and accumulators, f32 output.
//
// Semantics follow crates/tensor/src/ops/attention.rs:68-243 (online softmax
// over key tiles, causal mask j <= i [+ offset], out = acc * (1/l), or 0 when
// l == 0). The arithmetic differs only in summation order and in rounding the
// softmax weights to f16 before the PV product; the row sum l accumulates the
// same rounded weights, so the output is an exact convex combination of V rows
// with the rounded weights.
//
// Work decomposition: one workgroup = 4 waves = 256 queries of one
// (window, head); each wave owns two 32-query blocks. Per 64-key tile:
//   S^T[64 keys x 64 q] = K_tile[64 x 64] . Q^T      (4 x 4 MFMA 32x32x16)
//   O^T[64 d x 64 q]   += V_tile^T[64 x 64] . P^T    (4 x 4 MFMA 32x32x16 f16)
// Every K and V^T operand read from LDS feeds the MFMAs of both query blocks,
// which halves LDS read traffic per FLOP against one block per wave.
// Computing S^T (keys on the MFMA M axis) puts one query per lane, so the row
// max / row sum are register reductions plus one swap with lane^32, and the
// S^T accumulator registers are, after exp2 and packing, exactly the B operand
// of the PV product. V stays row-major in LDS; the transposed A operand of the
// PV product comes from ds_read_b64_tr_b16.
//
// Pipeline: K/V tiles are triple-buffered in LDS and the loop is software
// pipelined over 32-key half tiles, so each wave always has independent MFMA
// and VALU work: while the VALU computes the softmax weights of half h, the
// MFMAs of the next half's S^T run, followed by the PV MFMAs of half h. Tile
// t+2 (in registers) is written to the third buffer and the global loads of
// tile t+3 are in flight; one barrier per 64-key tile.
//
// Softmax rescaling is lazy: a query's reference max m only moves when a half
// tile raises the row max by more than 2^8 (in the exp2 domain), so most
// steps skip the O and l rescale. Weights exp2(x - m) then stay below 2^8, well inside the
// f16 range of the PV operand, and the final 1/l normalization is unchanged.
#include "wrs_internal.hpp"

namespace wrs {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kQB = 2;         // 32-query blocks per wave
constexpr int kM = 128 * kQB;  // queries per workgroup
constexpr int kN = 64;         // keys per tile
constexpr int kThreads = 256;  // 4 waves of 64
constexpr int kP = 72;         // LDS row pitch of the K and V tiles, in 16-bit elements
constexpr int kTile = kN * kP;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;  // rescale threshold, log2 units

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
      const f32x2 w = {__builtin_bit_cast(float, x[i] << 16),
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

// max / sum with the partner lane l ^ 32 (the other half of the same query).
// (ds_bpermute via __shfl_xor: this toolchain miscompiles
// __builtin_amdgcn_permlane32_swap when both operands are the same value.)
__device__ inline float pair_max(float x) { return fmaxf(x, __shfl_xor(x, 32)); }
__device__ inline float pair_sum(float x) { return x + __shfl_xor(x, 32); }

// Four consecutive keys of one d column, from a row-major [key][d] LDS tile.
__device__ inline u32x2 read_tr(const uint16_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4*)(reinterpret_cast<uintptr_t>(p)));
  return __builtin_bit_cast(u32x2, v);
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
  __shared__ __attribute__((aligned(16))) uint16_t Ks[3 * kTile];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[3 * kTile];

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

  // This lane's queries: column r32 of each of the wave's S^T blocks.
  int qi[kQB], qpos[kQB];
  u32x4 qf[kQB][4];
#pragma unroll
  for (int j = 0; j < kQB; ++j) {
    qi[j] = qblk * kM + wave * 32 * kQB + 32 * j + r32;
    qpos[j] = qi[j] + a.q_pos_offset;
    if (qi[j] < a.t_q) {
      const T* row = qp + static_cast<int64_t>(qi[j]) * a.lq.rs + hl * 8;
#pragma unroll
      for (int dk = 0; dk < 4; ++dk) qf[j][dk] = *reinterpret_cast<const u32x4*>(row + dk * 16);
    } else {
#pragma unroll
      for (int dk = 0; dk < 4; ++dk) qf[j][dk] = u32x4{0, 0, 0, 0};
    }
  }

  int kv_end = a.t_kv;
  if (a.causal) {
    // No query of this block reaches past its last row (attention.rs:132-134).
    const int last = min(qblk * kM + kM, a.t_q) - 1 + a.q_pos_offset;
    kv_end = min(kv_end, last + 1);
  }
  const int n_tiles = (kv_end + kN - 1) / kN;
  // Tiles that need no mask: every key < t_kv and, if causal, every key at or
  // before the first query of the block.
  int n_full = a.t_kv / kN;
  if (a.causal) n_full = min(n_full, (qblk * kM + a.q_pos_offset + 1) / kN);
  n_full = min(n_full, n_tiles);

  // Cooperative tile copy: thread owns 16-byte chunks (key ci/8, columns 8*(ci%8)).
  u32x4 kreg[2], vreg[2];
  auto load_tile = [&](int t) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int ci = tid + r * kThreads;
      const int key = t * kN + (ci >> 3), col = (ci & 7) * 8;
      kreg[r] = vreg[r] = u32x4{0, 0, 0, 0};
      if (key < a.t_kv) {
        kreg[r] = *reinterpret_cast<const u32x4*>(kp + static_cast<int64_t>(key) * a.lk.rs + col);
        vreg[r] = *reinterpret_cast<const u32x4*>(vp + static_cast<int64_t>(key) * a.lv.rs + col);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int ci = tid + r * kThreads;
      const int off = buf * kTile + (ci >> 3) * kP + (ci & 7) * 8;
      *reinterpret_cast<u32x4*>(Ks + off) = kreg[r];
      *reinterpret_cast<u32x4*>(Vs + off) = Elem<T>::to_f16(vreg[r]);
    }
  };

  // K A-operands of half h2 of the tile in buffer buf, and S^T = K Q^T for
  // those 32 keys and both query blocks.
  typedef f32x16 SBlk[kQB];
  auto kfetch = [&](int buf, int h2, u32x4 (&ka)[4]) {
    const uint16_t* kt = Ks + buf * kTile + (32 * h2 + r32) * kP + hl * 8;
#pragma unroll
    for (int dk = 0; dk < 4; ++dk) ka[dk] = *reinterpret_cast<const u32x4*>(kt + dk * 16);
  };
  auto qk = [&](const u32x4 (&ka)[4], SBlk& s) {
#pragma unroll
    for (int j = 0; j < kQB; ++j) s[j] = f32x16{};
#pragma unroll
    for (int dk = 0; dk < 4; ++dk)
#pragma unroll
      for (int j = 0; j < kQB; ++j) s[j] = Elem<T>::mfma(ka[dk], qf[j][dk], s[j]);
  };

  const float c = a.scale * kLog2e;  // exp(scale*s - m') == exp2(c*s - c*m)
  f32x16 o[kQB][2];                  // O^T rows d 0..31 / 32..63, column = query
  float m[kQB], l[kQB];              // reference max (exp2 domain), partial row sum
#pragma unroll
  for (int j = 0; j < kQB; ++j) {
    o[j][0] = o[j][1] = f32x16{};
    m[j] = -INFINITY;
    l[j] = 0.f;
  }

  // Accumulator register i of a 32x32 block holds key 8*(i/4) + 4*hl + i%4 of
  // its 32-key half.
  auto mask_half = [&](int t, int h2, SBlk& s) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kr = t * kN + 32 * h2 + 8 * (i >> 2) + 4 * hl + (i & 3);
#pragma unroll
      for (int j = 0; j < kQB; ++j)
        if (kr >= a.t_kv || (a.causal && kr > qpos[j])) s[j][i] = -INFINITY;
    }
  };
  // Row max of a half tile in the exp2 domain; if it exceeds the reference max
  // by more than kLazy, move the reference and rescale what is accumulated.
  auto rescale_for = [&](const SBlk& s) {
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      float mr = fmaxf(s[j][0], s[j][1]);
#pragma unroll
      for (int i = 2; i < 16; i += 2) mr = fmaxf(fmaxf(mr, s[j][i]), s[j][i + 1]);  // v_max3
      const float mx = pair_max(mr) * c;
      if (mx > m[j] + kLazy) {
        const float alpha = __builtin_amdgcn_exp2f(m[j] - mx);  // m == -inf -> 0
        m[j] = mx;
        l[j] *= alpha;
        o[j][0] *= alpha;
        o[j][1] *= alpha;
      }
    }
  };
  // P = exp2(c*S - m) in f16 and O^T += V^T P^T.
  // P^T is already in B-operand order: PV block kb2 covers tile keys
  // 16*kb2 + 8*(j/4) + 4*hl + j%4 for element j. V^T rows come from the
  // transposed read: lane group g = lane/16 reads rows 16*kb2 + 4*(g/2) [+8]
  // + (lane%16)/4 at columns 32*db + 16*(g%2) + 4*(lane%4), so lane
  // (d = 32*db + r32, hl) receives keys 16*kb2 + 4*hl + {0..3} [+8].
  const int g = lane >> 4, t4 = lane & 15;
  const int vlane = (4 * (g >> 1) + (t4 >> 2)) * kP + 16 * (g & 1) + 4 * (t4 & 3);
  auto vfetch = [&](int buf, int h2, u32x2 (&va)[8]) {
    const uint16_t* vrow = Vs + buf * kTile + vlane + 32 * h2 * kP;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const uint16_t* v0 = vrow + 16 * k2 * kP;
      va[4 * k2 + 0] = read_tr(v0);
      va[4 * k2 + 1] = read_tr(v0 + 8 * kP);
      va[4 * k2 + 2] = read_tr(v0 + 32);
      va[4 * k2 + 3] = read_tr(v0 + 8 * kP + 32);
    }
  };
  auto weights = [&](const SBlk& s, u32x4 (&pb)[kQB][2]) {
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      float ls = 0.f;
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const f32x2 pp = {
              __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][8 * k2 + 2 * w], c, -m[j])),
              __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][8 * k2 + 2 * w + 1], c, -m[j]))};
          const f16x2 hp = __builtin_convertvector(pp, f16x2);
          ls = __builtin_amdgcn_fdot2(hp, f16x2{1.0f16, 1.0f16}, ls, false);
          pb[j][k2][w] = __builtin_bit_cast(uint32_t, hp);
        }
      }
      l[j] += ls;
    }
  };
  auto pv = [&](const u32x2 (&va)[8], const u32x4 (&pb)[kQB][2]) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const u32x4 v0 = {va[4 * k2].x, va[4 * k2].y, va[4 * k2 + 1].x, va[4 * k2 + 1].y};
      const u32x4 v1 = {va[4 * k2 + 2].x, va[4 * k2 + 2].y, va[4 * k2 + 3].x, va[4 * k2 + 3].y};
#pragma unroll
      for (int j = 0; j < kQB; ++j) {
        o[j][0] = mfma_f16(v0, pb[j][k2], o[j][0]);
        o[j][1] = mfma_f16(v1, pb[j][k2], o[j][1]);
      }
    }
  };
  // One half step, in issue order: S^T MFMAs of the next half (K operands
  // already in registers), V^T reads and softmax weights of this half (the
  // VALU work overlaps those MFMAs), PV MFMAs of this half, K operands two
  // halves ahead. The caller then reduces the next half's row max (its MFMAs
  // have long finished) while the PV MFMAs drain.
  auto half_step = [&](int buf, int h2, const SBlk& s, u32x4 (&ka)[4], int kbuf, int kh2,
                       bool fetch_k, SBlk& n) {
    qk(ka, n);
    __builtin_amdgcn_sched_barrier(0);
    u32x2 va[8];
    vfetch(buf, h2, va);
    u32x4 pb[kQB][2];
    weights(s, pb);
    __builtin_amdgcn_sched_barrier(0);
    pv(va, pb);
    if (fetch_k) kfetch(kbuf, kh2, ka);
    __builtin_amdgcn_sched_barrier(0);
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
    if (n_tiles > 1) {
      load_tile(1);
      store_tile(1);
      if (n_tiles > 2) load_tile(2);
    }
    __syncthreads();
    u32x4 ka[4];
    kfetch(0, 0, ka);
    SBlk s, n;
    qk(ka, s);
    if (n_full == 0) mask_half(0, 0, s);
    rescale_for(s);
    kfetch(0, 1, ka);
    int t = 0;
    // Main loop: tiles t and t+1 both unmasked (and t+1 already in LDS).
    for (; t + 1 < n_full; ++t) {
      if (t + 2 < n_tiles) {
        store_tile((t + 2) % 3);
        if (t + 3 < n_tiles) load_tile(t + 3);
      }
      const int buf = t % 3, nbuf = (t + 1) % 3;
      half_step(buf, 0, s, ka, nbuf, 0, true, n);  // S of (t, 1); K of (t+1, 0)
      rescale_for(n);
      half_step(buf, 1, n, ka, nbuf, 1, true, s);  // S of (t+1, 0); K of (t+1, 1)
      rescale_for(s);
      __syncthreads();
    }
    // Tail: the last unmasked tile and the masked ones.
    for (; t < n_tiles; ++t) {
      if (t + 2 < n_tiles) {
        store_tile((t + 2) % 3);
        if (t + 3 < n_tiles) load_tile(t + 3);
      }
      const int buf = t % 3, nbuf = (t + 1) % 3;
      const bool has_next = t + 1 < n_tiles;
      half_step(buf, 0, s, ka, nbuf, 0, has_next, n);
      if (t >= n_full) mask_half(t, 1, n);
      rescale_for(n);
      half_step(buf, 1, n, ka, nbuf, 1, has_next, s);
      if (has_next) {
        if (t + 1 >= n_full) mask_half(t + 1, 0, s);
        rescale_for(s);
      }
      __syncthreads();
    }
  }

#pragma unroll
  for (int j = 0; j < kQB; ++j) {
    l[j] = pair_sum(l[j]);
    const float inv = (l[j] > 0.f) ? 1.f / l[j] : 0.f;
    if (qi[j] < a.t_q) {
      float* op = a.o + b * a.lo.bs + h * a.lo.hs + static_cast<int64_t>(qi[j]) * a.lo.rs;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        *reinterpret_cast<f32x4*>(op + 8 * gq + 4 * hl) =
            f32x4{o[j][0][4 * gq], o[j][0][4 * gq + 1], o[j][0][4 * gq + 2], o[j][0][4 * gq + 3]} *
            inv;
        *reinterpret_cast<f32x4*>(op + 32 + 8 * gq + 4 * hl) =
            f32x4{o[j][1][4 * gq], o[j][1][4 * gq + 1], o[j][1][4 * gq + 2], o[j][1][4 * gq + 3]} *
            inv;
      }
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
