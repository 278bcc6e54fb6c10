// Decode-step attention: one new query row per beam / slot against cached K/V.
//
// K2 (decode_f16): split-K attention over the f16 KV cache
//   (replaces crates/tensor/src/ops/attention.rs:246-434 single_token_mha_d64
//    as called from crates/whisper/src/decoder.rs:636 / :698).
//   Grid (split, head, group). A workgroup of 8 waves owns kChunk = 128
//   consecutive keys (256 when that covers the whole sequence, so that no
//   merge is needed) of one (group, head) plane and ALL query rows of the
//   group (the beams of an utterance share the cross-attention plane, so it is
//   read once per step instead of once per beam). Each wave takes one 16-key
//   tile (two, 128 keys apart, in a 256-key workgroup: a 16-wave workgroup of
//   one tile each cost ~1.2 us more per launch at any length), and every lane
//   issues its q loads and its four 16-byte K/V loads per tile before any
//   arithmetic, so the whole layer's cache is in flight from the first
//   cycles. The arithmetic runs on the matrix pipe, in registers:
//   - scores: one 16x16x32 f16 MFMA tile S^T = K Q^T per 32 d. The K rows
//     are the A operand exactly as loaded (lane (c, g): key c, d 8g..8g+7).
//     q*scale*log2(e) is scaled by a power of two per row and split into f16
//     high and low parts, placed in B columns r and r+8; a row_ror-8 DPP adds
//     the two columns, so the scores carry ~2^-22 relative error, not f16's.
//   - softmax: the wave's keys' max and exp2 sum per row, over the lane's 4
//     values per tile and two cross-row moves.
//   - P V: V^T comes out of a 16x16x32 MFMA of the V rows against a 0/1
//     selection matrix (exact), already in the B layout of a 16x16x16 MFMA
//     whose A operand is P as produced by the score tile, again as high
//     (rows 0-7) and low (rows 8-15) f16 parts.
//   The waves' (max, sum, 16x64 partials) meet in LDS; thread (row, d) folds
//   them with the log-sum-exp rule.
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
//   decoder.rs:884). Rows come in groups that share a K/V base; row i of
//   group g sees keys [0, glen[g] + i * limit_step).
#include "wrs_internal.hpp"

namespace wrs {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;            // exact f32 decode
constexpr int kRedPitch = 68;            // LDS pitch (floats) of a wave's 16 output rows
constexpr int kQsPitch = 68;             // LDS pitch (floats) of the staged q rows
constexpr int kPart = 68;    // floats per partial row: m, l, 2 pad, acc[64]
constexpr int kCounterStride = 32;  // 128 bytes between merge counters
constexpr int kRawBuffer = 0x00020000;  // buffer resource word 3: raw, 32-bit data format
constexpr int kMaxSplitsMerge = 16;  // partial loads in flight per thread in the merge

// Cross-lane moves inside a row of 16 lanes (DPP): xor 1, xor 2, mirror-8, mirror-16,
// rotate by 8.
template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                0xF, 0xF, false));
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


__device__ inline float pow2(int e) { return __builtin_bit_cast(float, (e + 127) << 23); }

// Row statistics for the one-pass alignment-head capture: (max, sum) in the
// exp2 domain, the scores being q.k * scale * log2(e).
__device__ inline void store_lse(const DecodeArgs& a, int row, int h, float m, float l) {
  float* st = a.lse + 2 * (static_cast<int64_t>(h) * a.lse_rows + a.lse_row0 + row);
  st[0] = m;
  st[1] = l;
}
__device__ inline int clamp_exp(int e) { return e < -126 ? -126 : (e > 127 ? 127 : e); }

// x op x[lane ^ 32] and x op x[lane ^ 16] with the gfx950 lane-swap VALU
// instructions (no LDS round trip). Issued as inline asm on two distinct
// registers: the swap writes both operands.
__device__ inline void swap32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ inline void swap16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ inline float max_x16_x32(float x) {
  float a = x, b = x;
  swap16(a, b);  // a, b: x of this row and of the row 16 lanes away
  x = fmaxf(a, b);
  a = x;
  b = x;
  swap32(a, b);
  return fmaxf(a, b);
}
__device__ inline float sum_x16_x32(float x) {
  float a = x, b = x;
  swap16(a, b);
  x = a + b;
  a = x;
  b = x;
  swap32(a, b);
  return a + b;
}


// kMWaves waves of kTiles 16-key tiles each: 8 waves of one tile (128 keys,
// kDecodeChunk) in general, 8 waves of two (kDecodeChunkLong = 256 keys) when
// that covers the whole sequence, which then needs no split-K merge. Tile t of
// wave w covers keys 128t + 16w.. of the workgroup's chunk.
// kDS == 4 (launches of one split per plane): the plane's 64 output columns
// are dealt to 4 workgroups, each reading all of K (the scores and softmax,
// repeated in each) but only its 16 columns of V, and writing those columns.
// One-split self-decode planes are bound by how fast one CU takes in its
// rows; this spreads them over 4 CUs of one XCD without a merge.
template <int R, int kMWaves, int kTiles, int kDS = 1>
__global__ __launch_bounds__(64 * kMWaves) void decode_f16(DecodeArgs a) {
  static_assert(kMWaves >= kMaxRowsPerGroup, "one merging wave per query row");
  static_assert(kMWaves == 8, "tile t of wave w starts at key 128t + 16w");
  constexpr int kChunk = 16 * kMWaves * kTiles;
  __shared__ float red[kMWaves][16][kRedPitch];
  __shared__ float wm[kMWaves][8], wl[kMWaves][8];
  __shared__ int last_flag;

  static_assert(kDS == 1 || kDS == 4, "whole or quarter rows of V");
  // kDS > 1: a 1-D grid of planes x parts, remapped so that a plane's parts
  // are neighbours on one XCD (their K reads meet in its L2).
  const int lid = kDS > 1 ? xcd_remap(blockIdx.x, gridDim.x) : 0;
  const int split = kDS > 1 ? 0 : blockIdx.x;
  const int h = kDS > 1 ? (lid / kDS) % a.n_heads : blockIdx.y;
  const int g = kDS > 1 ? (lid / kDS) / a.n_heads : blockIdx.z;
  const int dpart = kDS > 1 ? lid % kDS : 0;  // columns [64/kDS dpart, 64/kDS (dpart+1))
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  constexpr int rows = R;  // == a.rows_per_group
  const int len = a.len[g];
  const int col = lane & 15, kg = lane >> 4;
  const bool lo_part = col >= 8;

  // q * scale * log2(e), scaled per row by the power of two that puts the
  // row's largest magnitude into [2^14, 2^15). Groups of several rows (the
  // beams of a cross decode) stage it once per workgroup: thread t < rows*16
  // loads 4 values of row t/16 and stores them scaled in LDS. A one-row group
  // (a self-decode slot) has each lane load its own 16 values instead: the
  // staging barrier would hold back the workgroup's waves, which for short
  // sequences finish their keys soon after the loads land.
  constexpr bool kStageQ = rows > 1;
  const int qrow = col & 7;
  // Rows padded to 68 floats: the 8 rows read at one column fall in distinct
  // banks (at a 64-float pitch they shared them).
  __shared__ __attribute__((aligned(16))) float qs[kStageQ ? 8 : 1][kQsPitch];
  __shared__ float qdown[8];
  const bool qload = kStageQ && tid < rows * 16;
  f32x4 qx = {0.f, 0.f, 0.f, 0.f};
  float qv[16];
  if constexpr (kStageQ) {
    if (qload)
      qx = *reinterpret_cast<const f32x4*>(a.q + static_cast<int64_t>(g * rows + (tid >> 4)) *
                                                     a.q_rs + h * 64 + 4 * (tid & 15));
  } else {
    const float* qp = a.q + static_cast<int64_t>(g) * a.q_rs + h * 64 + 8 * kg;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qv[j] = qp[j];
      qv[8 + j] = qp[32 + j];
    }
  }
  // Lane (col, kg) carries key kbase + col: d 8kg..8kg+7 and 32+8kg.. of its
  // K and V rows (the A-operand layout of a 16x16x32 MFMA).
  const int kbase = split * kChunk + wave * 16;
  // The loads go through buffer resources whose range is the group's visible
  // rows: lanes past the length read zero without touching memory (an empty
  // or absent plane is never dereferenced), and no branch stands between the
  // loads and their use (a predicated form made the compiler wait for them
  // right away: +0.65 us per cross-decode launch).
  const int64_t plane = a.goff[g] + h * a.kv_hs;
  const uint32_t range = static_cast<uint32_t>(len) * 128u;
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(a.k + plane), 0, range, kRawBuffer);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(a.v + plane), 0, range, kRawBuffer);
  u32x4 kx0[kTiles], kx1[kTiles], vx0[kTiles], vx1[kTiles];
  // kDS == 4: vx0 holds the V half with the workgroup's 16 columns (d 32 hv +
  // 8 kg ..); lanes whose 8 columns lie outside them read zero through an
  // offset past the buffer's range (no memory access).
  const int hv = dpart >> 1;
  const bool vneed = (kg >> 1) == (dpart & 1);
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
    const uint32_t voff = static_cast<uint32_t>(kbase + 128 * tt + col) * 128u + 16u * kg;
    kx0[tt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, voff, 0, 0));
    kx1[tt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, voff + 64, 0, 0));
    if constexpr (kDS == 1) {
      vx0[tt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff, 0, 0));
      vx1[tt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff + 64, 0, 0));
    } else {
      const uint32_t vo = vneed ? voff + 64u * hv : 0xFFFFFFF0u;
      vx0[tt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vo, 0, 0));
      vx1[tt] = vx0[tt];
    }
  }
  // Every load above is issued before any of them is waited on: the q
  // arithmetic below depends on a value defined after them.
  float one;
  __asm__ volatile("v_mov_b32 %0, 1.0" : "=v"(one) : : "memory");
  float down;
  if constexpr (kStageQ) {
    if (qload) {
      qx *= a.scale_log2 * one;
      float amax = fmaxf(fmaxf(fabsf(qx[0]), fabsf(qx[1])), fmaxf(fabsf(qx[2]), fabsf(qx[3])));
      amax = fmaxf(amax, dpp<0xB1>(amax));  // the row's 16 lanes (DPP inside a row)
      amax = fmaxf(amax, dpp<0x4E>(amax));
      amax = fmaxf(amax, dpp<0x141>(amax));
      amax = fmaxf(amax, dpp<0x140>(amax));
      const int e_max = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xFF);
      const int sh = e_max == 0 ? 0 : clamp_exp(141 - e_max);
      *reinterpret_cast<f32x4*>(&qs[tid >> 4][4 * (tid & 15)]) = qx * pow2(sh);
      if ((tid & 15) == 0) qdown[tid >> 4] = pow2(clamp_exp(-sh));
    }
    __syncthreads();
    // Rows past the group's are zero.
    down = qrow < rows ? qdown[qrow] : 1.f;
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    const f32x4 q0 = qrow < rows ? *reinterpret_cast<const f32x4*>(&qs[qrow][8 * kg]) : z4;
    const f32x4 q1 = qrow < rows ? *reinterpret_cast<const f32x4*>(&qs[qrow][8 * kg + 4]) : z4;
    const f32x4 q2 = qrow < rows ? *reinterpret_cast<const f32x4*>(&qs[qrow][32 + 8 * kg]) : z4;
    const f32x4 q3 = qrow < rows ? *reinterpret_cast<const f32x4*>(&qs[qrow][36 + 8 * kg]) : z4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qv[j] = q0[j];
      qv[4 + j] = q1[j];
      qv[8 + j] = q2[j];
      qv[12 + j] = q3[j];
    }
  } else {
    // The one row sits in the B columns col == 0 (high) and 8 (low).
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      qv[j] = (qrow == 0 ? qv[j] : 0.f) * (a.scale_log2 * one);
      amax = fmaxf(amax, fabsf(qv[j]));
    }
    amax = max_x16_x32(amax);
    const int e_max = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xFF);
    const int sh = e_max == 0 ? 0 : clamp_exp(141 - e_max);
    const float up = pow2(sh);
#pragma unroll
    for (int j = 0; j < 16; ++j) qv[j] *= up;
    down = pow2(clamp_exp(-sh));
  }

  // Split into f16 high (columns 0-7 of B) and low (columns 8-15) parts.
  f16x8 b0, b1;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x0 = qv[j], x1 = qv[8 + j];
    const _Float16 h0 = static_cast<_Float16>(x0), h1 = static_cast<_Float16>(x1);
    b0[j] = lo_part ? static_cast<_Float16>(x0 - static_cast<float>(h0)) : h0;
    b1[j] = lo_part ? static_cast<_Float16>(x1 - static_cast<float>(h1)) : h1;
  }

  // S^T tile: lane (col, kg) gets keys kbase+4kg+i of column col; the high and
  // low columns of a row are eight lanes apart (row_ror 8 adds them).
  float sc[kTiles][4], mx = -INFINITY;
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, kx0[tt]), b0, s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, kx1[tt]), b1, s, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float si = s[i];
      const float full = (si + dpp<0x128>(si)) * down;
      sc[tt][i] = (kbase + 128 * tt + 4 * kg + i < len) ? full : -INFINITY;
      mx = fmaxf(mx, sc[tt][i]);
    }
  }
  mx = max_x16_x32(mx);
  float sum = 0.f;
  f16x4 pa[kTiles];
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sc[tt][i] - mx);
      sum += p;
      const _Float16 ph = static_cast<_Float16>(p);
      pa[tt][i] = lo_part ? static_cast<_Float16>(p - static_cast<float>(ph)) : ph;
    }
  sum = sum_x16_x32(sum);

  // V^T by multiplying with a 0/1 selection matrix (exact), then P V.
  f16x8 e0, e1;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    e0[j] = (8 * kg + j == col) ? static_cast<_Float16>(1.f) : static_cast<_Float16>(0.f);
    e1[j] = (8 * kg + j == 16 + col) ? static_cast<_Float16>(1.f) : static_cast<_Float16>(0.f);
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    // 16-column tile dt belongs to part dt / (4 / kDS).
    if (kDS > 1 && dt / (4 / kDS) != dpart) continue;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f32x4 o = z;
#pragma unroll
    for (int tt = 0; tt < kTiles; ++tt) {
      const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(f16x8, dt < 2 || kDS > 1 ? vx0[tt] : vx1[tt]), (dt & 1) ? e1 : e0, z,
          0, 0, 0);
      const f16x4 vb = __builtin_convertvector(t, f16x4);
      o = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[tt], vb, o, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][4 * kg + i][16 * dt + col] = o[i];
  }
  if (kg == 0 && col < 8) {
    wm[wave][col] = mx;
    wl[wave][col] = sum;
  }
  __syncthreads();

  // Thread (row qr, d qd) of the first rows*64 threads folds the waves'
  // partials (log-sum-exp, exp2 domain); rows r and r+8 are the high and low
  // parts of the weights.
  const int qr = tid >> 6, qd = kDS > 1 ? (64 / kDS) * dpart + (tid & 63) : tid & 63;
  const bool own = qr < rows && (kDS == 1 || (tid & 63) < 64 / kDS);
  float pv = 0.f, M = -INFINITY, Lsum = 0.f;
  if (own) {
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) M = fmaxf(M, wm[w][qr]);
    // Waves without a visible key hold m = -inf, l = 0 and zero partials.
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) {
      const float mw = wm[w][qr];
      const float al = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
      Lsum = __builtin_fmaf(wl[w][qr], al, Lsum);
      pv = __builtin_fmaf(red[w][qr][qd] + red[w][qr + 8][qd], al, pv);
    }
  }
  if (a.n_splits == 1) {
    if (own) {
      a.o[static_cast<int64_t>(g * rows + qr) * a.o_rs + h * 64 + qd] = Lsum > 0.f ? pv * (1.f / Lsum) : 0.f;
      if (a.lse && qd == 0) store_lse(a, g * rows + qr, h, M, Lsum);  // part 0 only
    }
    return;
  }

  const int gh = g * a.n_heads + h;
  float* mine = a.part + (static_cast<int64_t>(gh) * a.n_splits + split) * rows * kPart;
  if (own) st_agent(mine + qr * kPart + 4 + qd, pv);
  if (own && qd == 0) {
    st_agent(mine + qr * kPart, M);
    st_agent(mine + qr * kPart + 1, Lsum);
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
    if (a.lse && qd == 0) store_lse(a, g * rows + qr, h, M, L);
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

  const int g = row / a.rows_per_group;
  const int L = a.glen[g] + (row - g * a.rows_per_group) * a.limit_step;
  const int64_t kv0 = a.goff[g] + h * a.kv_hs;
  float* sc = a.scores + (static_cast<int64_t>(row) * a.n_heads + h) * a.scores_stride;
  float lmax = -INFINITY;
  for (int j = tid; j < L; j += kThreads) {
    const float* kr = a.k + kv0 + static_cast<int64_t>(j) * a.kv_rs;
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
        acc = __builtin_fmaf(w, a.v[kv0 + static_cast<int64_t>(j) * a.kv_rs + d], acc);
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

// Streaming read with the decode grid's shape: 512 threads x 64 bytes per
// workgroup, every load issued before any is used; one float per workgroup
// keeps the loads live.
__global__ __launch_bounds__(512) void stream_read(const u32x4* src, int64_t n16, float* sink) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 2048 + threadIdx.x;
  u32x4 x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t idx = base + 512 * i;
    x[i] = idx < n16 ? src[idx] : u32x4{0, 0, 0, 0};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) acc ^= x[i].x ^ x[i].y ^ x[i].z ^ x[i].w;
  __shared__ uint32_t red[8];
  for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int w = 0; w < 8; ++w) r ^= red[w];
    sink[blockIdx.x] = __builtin_bit_cast(float, r & 0x3fffffffu);
  }
}

// The same with a chosen shape: T threads per workgroup, L 16-byte loads per
// lane (lane i of workgroup b reads chunks b*T*L + i + T*j), all issued before
// any is used.
template <int T, int L>
__global__ __launch_bounds__(T) void stream_read_shape(const u32x4* src, int64_t n16, float* sink) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * T * L + threadIdx.x;
  u32x4 x[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const int64_t idx = base + static_cast<int64_t>(T) * i;
    x[i] = idx < n16 ? src[idx] : u32x4{0, 0, 0, 0};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < L; ++i) acc ^= x[i].x ^ x[i].y ^ x[i].z ^ x[i].w;
  __shared__ uint32_t red[T / 64];
  for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int w = 0; w < T / 64; ++w) r ^= red[w];
    sink[blockIdx.x] = __builtin_bit_cast(float, r & 0x3fffffffu);
  }
}

}  // namespace

int64_t stream_read_shape_blocks(int64_t bytes, int threads, int loads) {
  const int64_t per = static_cast<int64_t>(threads) * loads;
  return per > 0 ? (bytes / 16 + per - 1) / per : 0;
}

hipError_t launch_stream_read_shape(const void* src, int64_t bytes, int threads, int loads,
                                    float* sink, hipStream_t s) {
  const int64_t n16 = bytes / 16;
  const int64_t blocks = stream_read_shape_blocks(bytes, threads, loads);
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(blocks));
  const u32x4* p = static_cast<const u32x4*>(src);
#define WRS_SRS(T, L)                                                             \
  if (threads == T && loads == L) {                                               \
    hipLaunchKernelGGL((stream_read_shape<T, L>), grid, dim3(T), 0, s, p, n16, sink); \
    return hipGetLastError();                                                     \
  }
  WRS_SRS(256, 1) WRS_SRS(256, 2) WRS_SRS(256, 4) WRS_SRS(256, 8) WRS_SRS(256, 16) WRS_SRS(256, 24)
  WRS_SRS(512, 1) WRS_SRS(512, 2) WRS_SRS(512, 4) WRS_SRS(512, 8) WRS_SRS(512, 16) WRS_SRS(512, 24)
  WRS_SRS(1024, 1) WRS_SRS(1024, 2) WRS_SRS(1024, 4) WRS_SRS(1024, 8) WRS_SRS(1024, 16)
  WRS_SRS(1024, 24)
#undef WRS_SRS
  return hipErrorInvalidValue;
}

hipError_t launch_stream_read(const void* src, int64_t bytes, float* sink, hipStream_t s) {
  const int64_t n16 = bytes / 16;
  const int64_t blocks = (n16 + 2047) / 2048;
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(stream_read, dim3(static_cast<unsigned>(blocks)), dim3(512), 0, s,
                     static_cast<const u32x4*>(src), n16, sink);
  return hipGetLastError();
}

int64_t stream_read_blocks(int64_t bytes) { return (bytes / 16 + 2047) / 2048; }

size_t decode_part_floats(int n_groups, int n_heads, int n_splits, int rows) {
  return static_cast<size_t>(n_groups) * n_heads * n_splits * rows * kPart;
}

size_t decode_counter_words(int n_groups, int n_heads) {
  return static_cast<size_t>(n_groups) * n_heads * kCounterStride;
}

// CUs of the current device, read once.
int decode_cus() {
  static const int cus = [] {
    int dev = 0, n = 256;
    if (hipGetDevice(&dev) == hipSuccess)
      (void)hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    return n;
  }();
  return cus;
}

hipError_t launch_decode_f16(const DecodeArgs& a, hipStream_t s) {
  if (a.n_groups <= 0 || a.n_splits <= 0) return hipSuccess;
  if (a.chunk != kDecodeChunk && a.chunk != kDecodeChunkLong) return hipErrorInvalidValue;
  static_assert(kDecodeChunk == 128 && kDecodeChunkLong == 256, "8 waves of one or two tiles");
  const bool lng = a.chunk == kDecodeChunkLong;
  const int64_t planes = static_cast<int64_t>(a.n_groups) * a.n_heads;
  if (a.rows_per_group == 1 && lng && a.n_splits == 1 && 4 * planes <= decode_cus()) {
    // One-row planes of 129-256 keys (self decode) on a quarter of the CUs or
    // fewer: their V columns over 4 workgroups each. Same-box A/B, whisper-small
    // 5 slots x 12 heads: 4.69 against 4.78 us at 224 keys, 4.87 against
    // 4.98 at 256; halves, or quarters at 128 keys and below, were slower.
    const dim3 grid(static_cast<unsigned>(4 * planes)), block(512);
    hipLaunchKernelGGL((decode_f16<1, 8, 2, 4>), grid, block, 0, s, a);
    return hipGetLastError();
  }
  const dim3 grid(a.n_splits, a.n_heads, a.n_groups), block(512);
#define WRS_DEC(R)                                                          \
  if (lng)                                                                  \
    hipLaunchKernelGGL((decode_f16<R, 8, 2>), grid, block, 0, s, a);        \
  else                                                                      \
    hipLaunchKernelGGL((decode_f16<R, 8, 1>), grid, block, 0, s, a);
  switch (a.rows_per_group) {
    case 1: WRS_DEC(1) break;
    case 2: WRS_DEC(2) break;
    case 3: WRS_DEC(3) break;
    case 4: WRS_DEC(4) break;
    case 5: WRS_DEC(5) break;
    case 6: WRS_DEC(6) break;
    case 7: WRS_DEC(7) break;
    case 8: WRS_DEC(8) break;
    default: return hipErrorInvalidValue;
  }
#undef WRS_DEC
  return hipGetLastError();
}

hipError_t launch_decode_exact_f32(const ExactArgs& a, hipStream_t s) {
  if (a.n_rows <= 0 || a.n_heads <= 0) return hipSuccess;
  if (a.rows_per_group <= 0 || a.n_groups <= 0 || a.n_groups > kMaxExactGroups ||
      static_cast<int64_t>(a.n_groups) * a.rows_per_group < a.n_rows || a.n_rows > 65535 ||
      a.d_head <= 0 || a.d_head > 128)
    return hipErrorInvalidValue;
  const dim3 grid(a.n_heads, a.n_rows), block(kThreads);
  hipLaunchKernelGGL(decode_exact_f32, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace wrs

