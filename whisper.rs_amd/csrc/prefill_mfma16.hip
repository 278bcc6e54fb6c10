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
// Work decomposition: one workgroup = 4 waves = 128 queries of one
// (window, head); each wave owns 32 queries. Per 64-key tile:
//   S^T[64 keys x 32 q] = K_tile[64 x 64] . Q^T      (2 x 4 MFMA 32x32x16)
//   O^T[64 d x 32 q]   += V_tile^T[64 x 64] . P^T    (2 x 4 MFMA 32x32x16 f16)
// Computing S^T (keys on the MFMA M axis) puts one query per lane, so the row
// max / row sum are register reductions plus one swap with lane^32, and the
// S^T accumulator registers are, after exp2 and packing, exactly the B operand
// of the PV product. V stays row-major in LDS; the transposed A operand of the
// PV product comes from ds_read_b64_tr_b16.
//
// Pipeline: K/V tiles are double-buffered in LDS. While tile t is computed,
// tile t+1 (already in registers) is written to the other buffer and the
// global loads of tile t+2 are in flight; one barrier per tile.
//
// Softmax rescaling is lazy: a query's reference max m only moves when a tile
// raises the row max by more than 2^8 (in the exp2 domain), so most tiles skip
// the O and l rescale. Weights exp2(x - m) then stay below 2^8, well inside the
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

constexpr int kM = 128;        // queries per workgroup (32 per wave)
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
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2 * kTile];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2 * kTile];

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

  const float c = a.scale * kLog2e;  // exp(scale*s - m') == exp2(c*s - c*m)
  f32x16 o0 = {}, o1 = {};           // O^T rows d 0..31 and 32..63, column = query
  float m = -INFINITY;               // reference max in the exp2 domain
  float l = 0.f;                     // running sum over this lane's key half

  auto tile = [&](int t, bool masked) {
    const int buf = t & 1;
    const uint16_t* kt = Ks + buf * kTile;
    const uint16_t* vt = Vs + buf * kTile;
    // S^T = K Q^T for tile keys [0, 32) and [32, 64).
    f32x16 s0 = {}, s1 = {};
#pragma unroll
    for (int dk = 0; dk < 4; ++dk) {
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(kt + r32 * kP + dk * 16 + hl * 8);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(kt + (32 + r32) * kP + dk * 16 + hl * 8);
      s0 = Elem<T>::mfma(a0, qf[dk], s0);
      s1 = Elem<T>::mfma(a1, qf[dk], s1);
    }
    // Accumulator register i of a 32x32 block holds key 8*(i/4) + 4*hl + i%4.
    if (masked) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kr = t * kN + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (kr >= a.t_kv || (a.causal && kr > qpos)) s0[i] = -INFINITY;
        if (kr + 32 >= a.t_kv || (a.causal && kr + 32 > qpos)) s1[i] = -INFINITY;
      }
    }
    float mr = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int i = 1; i < 16; ++i) mr = fmaxf(mr, fmaxf(s0[i], s1[i]));
    const float mx = pair_max(mr) * c;
    if (mx > m + kLazy) {
      const float alpha = __builtin_amdgcn_exp2f(m - mx);  // m == -inf -> 0
      m = mx;
      l *= alpha;
      o0 *= alpha;
      o1 *= alpha;
    }
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
        const f32x2 pp = {__builtin_amdgcn_exp2f(__builtin_fmaf(x0, c, -m)),
                          __builtin_amdgcn_exp2f(__builtin_fmaf(x1, c, -m))};
        const f16x2 hp = __builtin_convertvector(pp, f16x2);
        ls = __builtin_amdgcn_fdot2(hp, f16x2{1.0f16, 1.0f16}, ls, false);
        pb[kb2][w] = __builtin_bit_cast(uint32_t, hp);
      }
    }
    l += ls;
    // O^T += V^T P^T. Lane group g = lane/16 reads rows 16*kb2 + 4*(g/2) [+8]
    // + (lane%16)/4 at columns 32*db + 16*(g%2) + 4*(lane%4), so the transposed
    // read hands lane (d = 32*db + r32, hl) keys 16*kb2 + 4*hl + {0..3} [+8].
    const int g = lane >> 4, t4 = lane & 15;
    const uint16_t* vrow = vt + (4 * (g >> 1) + (t4 >> 2)) * kP + 16 * (g & 1) + 4 * (t4 & 3);
#pragma unroll
    for (int kb2 = 0; kb2 < 4; ++kb2) {
      const uint16_t* v0 = vrow + 16 * kb2 * kP;
      const u32x2 a0l = read_tr(v0), a0h = read_tr(v0 + 8 * kP);
      const u32x2 a1l = read_tr(v0 + 32), a1h = read_tr(v0 + 8 * kP + 32);
      o0 = mfma_f16(u32x4{a0l.x, a0l.y, a0h.x, a0h.y}, pb[kb2], o0);
      o1 = mfma_f16(u32x4{a1l.x, a1l.y, a1h.x, a1h.y}, pb[kb2], o1);
    }
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
    if (n_tiles > 1) load_tile(1);
    __syncthreads();
    for (int t = 0; t < n_tiles; ++t) {
      if (t + 1 < n_tiles) {
        store_tile((t + 1) & 1);
        if (t + 2 < n_tiles) load_tile(t + 2);
      }
      tile(t, t >= n_full);
      __syncthreads();
    }
  }

  l = pair_sum(l);
  const float inv = (l > 0.f) ? 1.f / l : 0.f;
  if (qi < a.t_q) {
    float* op = a.o + b * a.lo.bs + h * a.lo.hs + static_cast<int64_t>(qi) * a.lo.rs;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      *reinterpret_cast<f32x4*>(op + 8 * gq + 4 * hl) =
          f32x4{o0[4 * gq], o0[4 * gq + 1], o0[4 * gq + 2], o0[4 * gq + 3]} * inv;
      *reinterpret_cast<f32x4*>(op + 32 + 8 * gq + 4 * hl) =
          f32x4{o1[4 * gq], o1[4 * gq + 1], o1[4 * gq + 2], o1[4 * gq + 3]} * inv;
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
