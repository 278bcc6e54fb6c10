// Projections with f16 weights: out(t, r) = W[r] . x[t] + bias[r]
// (replaces crates/tensor/src/ops/quant.rs:415-473 f16_linear, reached through
//  LinearWeight::linear, crates/tensor/src/weight.rs:116-137, from the
//  encoder's fused QKV projection, crates/whisper/src/encoder.rs:275-277, and
//  the cross-attention K/V precompute, crates/whisper/src/decoder.rs:423-447).
//
// K6 (linear_f16w): D^T = W X^T on v_mfma_f32_32x32x16_f16. Both operands are
//   "k-contiguous" rows as stored (W [n_out][n_in] f16, X [n_tokens][k] f16),
//   so neither needs a transpose. A workgroup of 8 waves owns a tile of 256
//   output features x 256 tokens; wave (wm, wn) owns 128 x 64 of it as 4 x 2
//   MFMA tiles (6 operand reads per 8 MFMAs). k advances 64 per LDS stage
//   through two stages (128 KB): tiles move global -> LDS with
//   buffer_load ... lds (no staging registers), one stage ahead of the
//   MFMAs, and rows past the matrix edge read as zero through the buffer
//   range check; one barrier per stage (64-k stages halved the barriers of
//   the earlier 32-k, three-stage ring: 0.285 -> 0.267 ms). LDS rows (128
//   bytes) keep their 16-byte chunks XOR-permuted by the row index, so the 32
//   rows read by one operand fetch spread over the banks (swz_f). Workgroups are ordered so
//   that each XCD runs a compact block of 4 feature x 8 token tiles at a time.
//   Measured on the large-v3 fused QKV shape (24000 x 1280 x 3840): this
//   shape of tile reaches ~85% of the library GEMM on the same box.
//   f32 activations go to the f16 matrix pipe through a pre-pass
//   (linear_split_rows): each row is scaled by a power of two so that its
//   largest element lies in [2^14, 2^15), then split into two f16 parts
//   hi + lo that sum to it within 2^-22 relative (2^-25 of the row maximum
//   where lo is subnormal). The GEMM then runs over k' = 2 n_in with the
//   weight column k' mod n_in; each product carries at most that 2^-22
//   relative error, below what one f32 addition of the accumulation
//   (dot_f16_f32, simd.rs:593-700) already rounds away. The epilogue multiplies by
//   the row's 2^-shift (exact), adds the f32 bias and writes the output type
//   at out + t * out_rs + (r / 64) * out_hs + r % 64: token-major rows
//   (out_hs = 64) or the arena's [head][token][64] planes. A 16-bit tile
//   passes through the freed stage buffers first and leaves as whole 512-byte
//   token rows, 16 bytes per lane: stored straight from the MFMA layout (8
//   bytes of 32 different rows per instruction) the same bytes took 2.2x as
//   long to write. f32 output is stored straight from the MFMA layout.
#include "wrs_internal.hpp"

#include <algorithm>
#include <atomic>

namespace wrs {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4v __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 256;          // output features per workgroup (MFMA M)
constexpr int kBN = 256;          // tokens per workgroup (MFMA N)
constexpr int kBK = 64;           // k per LDS stage: one 128-byte row per feature/token
constexpr int kStages = 2;        // LDS ring
constexpr int kStageA = kBM * kBK;  // f16 elements per stage
constexpr int kStageB = kBN * kBK;
constexpr int kDmaA = kBM / kWaves / 8;  // 1 KB DMA instructions per wave per stage (4)
constexpr int kDmaB = kBN / kWaves / 8;  // (4)

// 16-byte chunk c of LDS row r sits at slot c ^ f(r), f(r) = (r >> 1) & 7.
// An operand fetch reads one chunk of 32 consecutive rows; 16 lanes at a time
// cover 256 bytes of banks, i.e. two 128-byte rows per bank line, so the 8
// even (and the 8 odd) rows of every 16 must land in distinct slots; f does
// that.
__device__ inline int swz_f(int row) { return (row >> 1) & 7; }
__device__ inline int swz(int row, int chunk) { return chunk ^ swz_f(row); }

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from global memory into LDS at m0 + 16 * lane, through a
// buffer resource (offsets past its size read as zero). Inline asm, so the
// compiler adds no waits of its own before later LDS reads; the kernel orders
// it with explicit vmcnt waits and barriers. m0 is used by nothing else here.
__device__ inline void dma16(u32x4 rsrc, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ inline u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000u;  // raw buffer, 32-bit data format
  return r;
}

__device__ inline uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// This wave's stage landed (no DMA load left in flight) and its LDS writes are
// done, then all waves meet.
__device__ inline void stage_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Physical workgroup id -> tile. The hardware hands linear ids round-robin to
// the 8 XCDs; each XCD is given a contiguous range of logical ids instead, and
// logical ids walk groups of kGroupM feature tiles with the token tiles
// outermost inside a group, so the ~32 workgroups an XCD runs at once cover
// 4 feature x 8 token tiles and share their operand stages in its L2.
constexpr int kGroupM = 4;
__device__ inline void tile_of(int pid, int n_fm, int n_tn, int& fm, int& tn) {
  const int nwg = n_fm * n_tn;
  const int xcd = pid & 7, k = pid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  const int id = xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
  const int group = id / (kGroupM * n_tn);
  const int gm = min(kGroupM, n_fm - group * kGroupM);
  const int in = id - group * kGroupM * n_tn;
  fm = group * kGroupM + in % gm;
  tn = in / gm;
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void linear_f16w(LinearArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 lds_ab[kStages * (kStageA + kStageB)];
  __shared__ __attribute__((aligned(16))) float bias_s[kBM];  // this tile's bias
  _Float16* const lds_a = lds_ab;
  _Float16* const lds_b = lds_ab + kStages * kStageA;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave & 1, wn = wave >> 1;  // 128-feature and 64-token block of this wave
  const int n_fm = (a.n_out + kBM - 1) / kBM, n_tn = (a.n_tokens + kBN - 1) / kBN;
  int fm, tn;
  tile_of(blockIdx.x, n_fm, n_tn, fm, tn);
  const int m0 = fm * kBM;  // first output feature
  const int n0 = tn * kBN;  // first token
  const int grp = blockIdx.z;

  // DMA sources. A wave moves rows 32*wave.. of the A and of the B tile, 16
  // rows per instruction; lane i lands at slot i%4 of row i/4 and so fetches
  // logical chunk swz(row, i%4). Rows past n_out / n_tokens fall
  // outside the buffer ranges and read as zero.
  const u32x4 wrs = buffer_rsrc(a.w[grp], static_cast<uint32_t>(
                                              static_cast<int64_t>(a.n_out) * a.n_in * 2));
  const u32x4 xrs = buffer_rsrc(
      a.x, static_cast<uint32_t>(((static_cast<int64_t>(a.n_tokens) - 1) * a.x_rs + a.k_total) *
                                 2));
  uint32_t aoff[kDmaA], boff[kDmaB];
#pragma unroll
  for (int j = 0; j < kDmaA; ++j) {
    const int row = wave * (kBM / kWaves) + 8 * j + (lane >> 3);
    const int ch = swz(row, lane & 7);
    aoff[j] = static_cast<uint32_t>((static_cast<int64_t>(m0 + row) * a.n_in + ch * 8) * 2);
  }
#pragma unroll
  for (int j = 0; j < kDmaB; ++j) {
    const int row = wave * (kBN / kWaves) + 8 * j + (lane >> 3);
    const int ch = swz(row, lane & 7);
    boff[j] = static_cast<uint32_t>((static_cast<int64_t>(n0 + row) * a.x_rs + ch * 8) * 2);
  }
  const uint32_t a_lds = lds_addr(lds_a) + wave * (kBM / kWaves) * kBK * 2;
  const uint32_t b_lds = lds_addr(lds_b) + wave * (kBN / kWaves) * kBK * 2;
  auto issue_stage = [&](int kt) {
    const uint32_t kx = static_cast<uint32_t>(kt * kBK * 2);             // x' column, bytes
    const uint32_t kw = static_cast<uint32_t>((kt * kBK) % a.n_in * 2);  // W column, bytes
    const int s = kt % kStages;
    const uint32_t ab = __builtin_amdgcn_readfirstlane(a_lds + s * kStageA * 2);
    const uint32_t bb = __builtin_amdgcn_readfirstlane(b_lds + s * kStageB * 2);
#pragma unroll
    for (int j = 0; j < kDmaA; ++j) dma16(wrs, ab + j * 1024, aoff[j] + kw);
#pragma unroll
    for (int j = 0; j < kDmaB; ++j) dma16(xrs, bb + j * 1024, boff[j] + kx);
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Operand rows of this lane: feature/token l % 32 of each 32-row MFMA tile,
  // k-group l / 32 (8 consecutive k) of each 16-k step.
  const int orow = lane & 31, kgrp = lane >> 5;
  int aread[4][kBK / 16], bread[2][kBK / 16];
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ra = wm * 128 + i * 32 + orow;
      aread[i][ks] = ra * kBK + swz(ra, 2 * ks + kgrp) * 8;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rb = wn * 64 + j * 32 + orow;
      bread[j][ks] = rb * kBK + swz(rb, 2 * ks + kgrp) * 8;
    }
  }

  const int n_kt = a.k_total / kBK;
  issue_stage(0);
  // The tile's bias goes to LDS while the first stage is in flight (the loop's
  // barriers order the write before the epilogue's reads): the epilogue then
  // reads it without a global-memory round trip per store.
  {
    const float* bias_g = a.bias[grp];
    if (threadIdx.x < kBM)
      bias_s[threadIdx.x] =
          (bias_g && m0 + static_cast<int>(threadIdx.x) < a.n_out) ? bias_g[m0 + threadIdx.x] : 0.0f;
  }
  for (int kt = 0; kt < n_kt; ++kt) {
    stage_barrier();
    if (kt + 1 < n_kt) issue_stage(kt + 1);  // its buffer was last read in step kt - 1
    const _Float16* as = lds_a + (kt % kStages) * kStageA;
    const _Float16* bs = lds_b + (kt % kStages) * kStageB;
    f16x8 av[kBK / 16][4], bv[kBK / 16][2];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
#pragma unroll
      for (int i = 0; i < 4; ++i) av[ks][i] = *reinterpret_cast<const f16x8*>(as + aread[i][ks]);
#pragma unroll
      for (int j = 0; j < 2; ++j) bv[ks][j] = *reinterpret_cast<const f16x8*>(bs + bread[j][ks]);
    }
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[ks][i], bv[ks][j], acc[i][j], 0, 0, 0);
  }

  // Epilogue: acc[i][j][e] is feature m0 + 64 wm + 32 i + 8 (e / 4) + 4 kgrp + e % 4
  // of token n0 + 64 wn + 32 j + orow.
  OutT* out = reinterpret_cast<OutT*>(a.out[grp]);
  const float* bias = a.bias[grp];
  if constexpr (sizeof(OutT) == 2) {
    // 16-bit output: the tile goes through LDS (the stage buffers, 128 KB:
    // 256 token rows of 512 bytes, 16-byte chunk c of row t at c ^ (t % 32)),
    // then leaves as whole rows: 64 lanes store 2 rows of 512 bytes.
    char* ot = reinterpret_cast<char*>(lds_a);  // lds_a and lds_b are one 128 KB span
    // this lane's 64 bias values, read before any LDS write of the tile, so
    // that no read waits behind the writes
    f32x4 bv[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        bv[i][g] = bias ? *reinterpret_cast<const f32x4*>(&bias_s[wm * 128 + i * 32 + 8 * g + 4 * kgrp])
                        : f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();                             // every wave is done with the last stage
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int tl = wn * 64 + j * 32 + orow;
      const int t = n0 + tl;
      const float rs = (a.row_scale && t < a.n_tokens) ? a.row_scale[t] : 1.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int fl = wm * 128 + i * 32 + 8 * g + 4 * kgrp;  // feature within the tile
          f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                     acc[i][j][4 * g + 3]};
          v *= rs;
          v += bv[i][g];
          if (a.act == kActGelu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
          }
          u32x2 h;
          if constexpr (__is_same(OutT, __bf16)) {
            typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
            h = __builtin_bit_cast(u32x2, __builtin_convertvector(v, bf16x4));
          } else {
            typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
            h = __builtin_bit_cast(u32x2, __builtin_convertvector(v, f16x4));
          }
          const int chunk = (fl >> 3) ^ (tl & 31);
          *reinterpret_cast<u32x2*>(ot + tl * 512 + chunk * 16 + (fl & 4) * 2) = h;
        }
    }
    __syncthreads();
    const bool v16 = ((reinterpret_cast<uintptr_t>(out) | (a.out_rs * 2) | (a.out_hs * 2)) & 15) == 0;
    const int c = lane & 31;  // 16-byte chunk: features 8c .. 8c + 7 of the row
    const int r = m0 + 8 * c;
    OutT* ocol = out + static_cast<int64_t>(r >> 6) * a.out_hs + (r & 63);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int tl = wave * 32 + 2 * q + (lane >> 5);
      const int t = n0 + tl;
      const u32x4 h = *reinterpret_cast<const u32x4*>(ot + tl * 512 + ((c ^ (tl & 31)) * 16));
      if (t < a.n_tokens && r < a.n_out) {
        OutT* p = ocol + static_cast<int64_t>(t) * a.out_rs;
        if (v16 && r + 8 <= a.n_out) {
          *reinterpret_cast<u32x4*>(p) = h;
        } else {
          *reinterpret_cast<u32x2*>(p) = u32x2{h[0], h[1]};
          if (r + 8 <= a.n_out) *reinterpret_cast<u32x2*>(p + 4) = u32x2{h[2], h[3]};
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = n0 + wn * 64 + j * 32 + orow;
      if (t >= a.n_tokens) continue;
      const float rs = a.row_scale ? a.row_scale[t] : 1.0f;
      OutT* orow_p = out + static_cast<int64_t>(t) * a.out_rs;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int r = m0 + wm * 128 + i * 32 + 8 * g + 4 * kgrp;
          if (r >= a.n_out) continue;
          f32x4 v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                     acc[i][j][4 * g + 3]};
          v *= rs;
          if (bias) v += *reinterpret_cast<const f32x4*>(&bias_s[r - m0]);
          if (a.act == kActGelu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
          }
          *reinterpret_cast<f32x4*>(orow_p + static_cast<int64_t>(r >> 6) * a.out_hs + (r & 63)) = v;
        }
    }
  }
}

// K7 (gemv_f16w): decode-sized batches (n_tokens <= 8: the beams of one step)
//   against f16 weights, f16_gemv_parallel semantics (quant.rs:343-413). The
//   weight stream is the whole cost, so every 16-byte chunk of W is read once
//   for all rows. One persistent workgroup of 8 waves per CU stages all of x
//   in LDS once (f32; f16 x widened exactly; at most kGemvXFloats values),
//   then its waves walk groups of 4 output features (1 when n_out <= 4096, so
//   that a d x d matrix still spreads over ~n_out / 8 CUs) across the matrix: lane l
//   multiplies W[r][k..k+8) for k = 8 l + 512 m by the staged x of every row
//   with f32 FMAs (the products dot_f16_f32 forms). The 16-byte loads of the
//   next 2048-column batch (or of the next group) are in flight while a batch
//   is multiplied. The row count is a template parameter (1..8), so no FMA is
//   issued for absent rows; the 64 lane partials reduce with DPP and two
//   cross-row moves, and lane b stores row b.
constexpr int kGemvWaves = 8;
constexpr int kGemvChunk = 2048;                // W columns per load batch
constexpr int kGemvSmallOut = 4096;             // one feature per wave up to this n_out
constexpr int kGemvSteps = kGemvChunk / 512;    // 16-byte W loads per row and batch

template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                0xF, 0xF, false));
}
// Sum over the 64 lanes: xor 1, xor 2 (quad perms), the mirror of each half row
// of 8 and of each row of 16 (DPP), then the two cross-row moves.
__device__ inline float wave_sum64(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

// LayerNorm of one f32 row by one wave, in the arithmetic of layer_norm_rows
// (elementwise.hip, norm.rs:116-143): lane partials over k = 4 lane + 256 i,
// mean, then the variance around it, each reduced with wave_sum64; so the
// normalized values equal that kernel's output bit for bit.
__device__ inline void ln_row_stats(const float* xr, int d, float eps, float& mean,
                                    float& inv_std) {
  const int lane = threadIdx.x & 63;
  float s = 0.0f;
  for (int k = 4 * lane; k < d; k += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(xr + k);
    s += (v[0] + v[1]) + (v[2] + v[3]);
  }
  mean = wave_sum64(s) / static_cast<float>(d);
  float q = 0.0f;
  for (int k = 4 * lane; k < d; k += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(xr + k);
#pragma unroll
    for (int j = 0; j < 4; ++j) q = fmaf(v[j] - mean, v[j] - mean, q);
  }
  const float var = wave_sum64(q) / static_cast<float>(d);
  inv_std = 1.0f / sqrtf(var + eps);
}
__device__ inline f32x4 ln_apply(const float* xr, const float* g, const float* b, int k,
                                 float mean, float inv_std) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(xr + k);
  const f32x4 gg = *reinterpret_cast<const f32x4*>(g + k);
  const f32x4 bb = *reinterpret_cast<const f32x4*>(b + k);
  f32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = fmaf((v[j] - mean) * inv_std, gg[j], bb[j]);
  return o;
}

// Rows of up to 256 * kLnCache values live in registers: lane l holds
// columns 4 l + 256 i in v[i] (zeros past d). The loads are issued first
// (ln_row_load), the arithmetic follows (ln_row_norm), with the arithmetic
// of ln_row_stats / ln_apply exactly.
constexpr int kLnCache = 5;  // 1280 columns: every Whisper d_model
__device__ inline void ln_row_load(const float* xr, const float* g, const float* b, int d,
                                   f32x4 (&v)[kLnCache], f32x4 (&gg)[kLnCache],
                                   f32x4 (&bb)[kLnCache]) {
  const int lane = threadIdx.x & 63;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kLnCache; ++i) {
    const int k = 4 * lane + 256 * i;
    const bool in = k < d;
    v[i] = in ? *reinterpret_cast<const f32x4*>(xr + k) : z;
    if (g) {
      gg[i] = in ? *reinterpret_cast<const f32x4*>(g + k) : z;
      bb[i] = in ? *reinterpret_cast<const f32x4*>(b + k) : z;
    }
  }
}
__device__ inline void ln_row_norm(int d, float eps, f32x4 (&v)[kLnCache],
                                   const f32x4 (&gg)[kLnCache], const f32x4 (&bb)[kLnCache]) {
  const int lane = threadIdx.x & 63;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kLnCache; ++i) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
  const float mean = wave_sum64(s) / static_cast<float>(d);
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < kLnCache; ++i) {
    if (4 * lane + 256 * i >= d) break;
#pragma unroll
    for (int j = 0; j < 4; ++j) q = fmaf(v[i][j] - mean, v[i][j] - mean, q);
  }
  const float var = wave_sum64(q) / static_cast<float>(d);
  const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < kLnCache; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) v[i][j] = fmaf((v[i][j] - mean) * inv_std, gg[i][j], bb[i][j]);
}

template <int NT, int kGemvRowsPerWave, typename XT, typename OutT>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_f16w(GemvArgs a) {
  __shared__ __attribute__((aligned(16))) float xs[kGemvXFloats];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int grp = blockIdx.y;
  const int n_in = a.n_in;
  const _Float16* w = a.w[grp];

  OutT* out = reinterpret_cast<OutT*>(a.out[grp]);
  const float* bias = a.bias[grp];
  const int n_groups4 = (a.n_out + kGemvRowsPerWave - 1) / kGemvRowsPerWave;
  const int stride = gridDim.x * kGemvWaves;
  // W loads of one 2048-column batch of one group of 4 features.
  auto load_w = [&](int g4, int c0, uint4 (&wv)[kGemvRowsPerWave][kGemvSteps]) {
#pragma unroll
    for (int i = 0; i < kGemvRowsPerWave; ++i) {
      const int r = min(g4 * kGemvRowsPerWave + i, a.n_out - 1);
      const _Float16* wr = w + static_cast<int64_t>(r) * n_in + c0;
#pragma unroll
      for (int m = 0; m < kGemvSteps; ++m) {
        const int k = 8 * lane + 512 * m;
        if (c0 + k < n_in) wv[i][m] = *reinterpret_cast<const uint4*>(wr + k);
      }
    }
  };
  int g4 = blockIdx.x * kGemvWaves + wave;
  uint4 wv[kGemvRowsPerWave][kGemvSteps];
  if (g4 < n_groups4) load_w(g4, 0, wv);  // in flight while x is staged

  // Stage x: row b at xs[b * n_in ..], 8 columns per thread and step, the
  // 16-byte loads of 4 steps in flight before their stores. With a fused
  // LayerNorm, wave b normalizes row b instead.
  if constexpr (sizeof(XT) == 4) {
    if (a.ln_g) {
      if (wave < NT) {
        const float* xr = static_cast<const float*>(a.x) + static_cast<int64_t>(wave) * a.x_rs;
        if (n_in <= 256 * kLnCache) {
          f32x4 y[kLnCache], gg[kLnCache], bb[kLnCache];
          ln_row_load(xr, a.ln_g, a.ln_b, n_in, y, gg, bb);
          ln_row_norm(n_in, a.ln_eps, y, gg, bb);
#pragma unroll
          for (int i = 0; i < kLnCache; ++i) {
            const int k = 4 * lane + 256 * i;
            if (k < n_in) *reinterpret_cast<f32x4*>(&xs[wave * n_in + k]) = y[i];
          }
        } else {
          float mean, inv_std;
          ln_row_stats(xr, n_in, a.ln_eps, mean, inv_std);
          for (int k = 4 * lane; k < n_in; k += 256)
            *reinterpret_cast<f32x4*>(&xs[wave * n_in + k]) =
                ln_apply(xr, a.ln_g, a.ln_b, k, mean, inv_std);
        }
      }
    }
  }
  if (!a.ln_g) {
    const int n8 = NT * n_in / 8;
    for (int e0 = tid; e0 < n8; e0 += 4 * 64 * kGemvWaves) {
      float v[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = e0 + u * 64 * kGemvWaves;
        if (e < n8) {
          const int b = (8 * e) / n_in, k = 8 * e - b * n_in;
          const XT* src = static_cast<const XT*>(a.x) + b * a.x_rs + k;
          if constexpr (sizeof(XT) == 4) {
            const float4 lo = *reinterpret_cast<const float4*>(src);
            const float4 hi = *reinterpret_cast<const float4*>(src + 4);
            v[u][0] = lo.x; v[u][1] = lo.y; v[u][2] = lo.z; v[u][3] = lo.w;
            v[u][4] = hi.x; v[u][5] = hi.y; v[u][6] = hi.z; v[u][7] = hi.w;
          } else {
            const f16x8 h = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(src));
#pragma unroll
            for (int j = 0; j < 8; ++j) v[u][j] = static_cast<float>(h[j]);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = e0 + u * 64 * kGemvWaves;
        if (e < n8) {
          *reinterpret_cast<float4*>(&xs[8 * e]) = float4{v[u][0], v[u][1], v[u][2], v[u][3]};
          *reinterpret_cast<float4*>(&xs[8 * e + 4]) = float4{v[u][4], v[u][5], v[u][6], v[u][7]};
        }
      }
    }
  }
  __syncthreads();

  for (; g4 < n_groups4; g4 += stride) {
    // The group's bias is loaded now, so that its latency hides under the
    // products instead of following the reduction.
    float bias_v[kGemvRowsPerWave];
#pragma unroll
    for (int i = 0; i < kGemvRowsPerWave; ++i) {
      const int r = min(g4 * kGemvRowsPerWave + i, a.n_out - 1);
      bias_v[i] = bias ? bias[r] : 0.0f;
    }
    float acc[kGemvRowsPerWave][NT];
#pragma unroll
    for (int i = 0; i < kGemvRowsPerWave; ++i)
#pragma unroll
      for (int b = 0; b < NT; ++b) acc[i][b] = 0.0f;
    for (int c0 = 0; c0 < n_in; c0 += kGemvChunk) {
      uint4 cur[kGemvRowsPerWave][kGemvSteps];
#pragma unroll
      for (int i = 0; i < kGemvRowsPerWave; ++i)
#pragma unroll
        for (int m = 0; m < kGemvSteps; ++m) cur[i][m] = wv[i][m];
      // the next batch (or the next group's first) is in flight during this one
      if (c0 + kGemvChunk < n_in)
        load_w(g4, c0 + kGemvChunk, wv);
      else if (g4 + stride < n_groups4)
        load_w(g4 + stride, 0, wv);
#pragma unroll
      for (int m = 0; m < kGemvSteps; ++m) {
        const int k = c0 + 8 * lane + 512 * m;
        if (k >= n_in) break;
        float xv[NT][8];
#pragma unroll
        for (int b = 0; b < NT; ++b) {
          const float4 lo = *reinterpret_cast<const float4*>(&xs[b * n_in + k]);
          const float4 hi = *reinterpret_cast<const float4*>(&xs[b * n_in + k + 4]);
          xv[b][0] = lo.x; xv[b][1] = lo.y; xv[b][2] = lo.z; xv[b][3] = lo.w;
          xv[b][4] = hi.x; xv[b][5] = hi.y; xv[b][6] = hi.z; xv[b][7] = hi.w;
        }
#pragma unroll
        for (int i = 0; i < kGemvRowsPerWave; ++i) {
          const f16x8 h = __builtin_bit_cast(f16x8, cur[i][m]);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float wf = static_cast<float>(h[j]);
#pragma unroll
            for (int b = 0; b < NT; ++b) acc[i][b] = fmaf(wf, xv[b][j], acc[i][b]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kGemvRowsPerWave; ++i)
#pragma unroll
      for (int b = 0; b < NT; ++b) acc[i][b] = wave_sum64(acc[i][b]);
    if (lane < NT) {
      const int r0 = g4 * kGemvRowsPerWave;
#pragma unroll
      for (int i = 0; i < kGemvRowsPerWave; ++i) {
        const int r = r0 + i;
        if (r >= a.n_out) break;
        float v = 0.0f;
#pragma unroll
        for (int b = 0; b < NT; ++b)
          if (b == lane) v = acc[i][b];
        if (bias) v += bias_v[i];
        if (a.act == kActGelu) v = gelu_tanh(v);
        out[static_cast<int64_t>(lane) * a.out_rs + static_cast<int64_t>(r >> 6) * a.out_hs +
            (r & 63)] = static_cast<OutT>(v);
      }
    }
  }
}

// K7m (gemv_f16w_mfma): the same product for 3..8 x rows on the matrix pipe.
//   W is read in tiles of T <= 16 features: lane (c, g) of a wave loads 16
//   bytes of feature c (columns 32 s + 8 g ..) per 32-column k-step s, which is
//   the A operand of a 16x16x32 f16 MFMA as loaded; lanes c >= T repeat the
//   tile's first feature (no extra traffic) and feed zeros. T = ceil(n_out /
//   n_CU) up to 16, so that a d x d matrix still spreads over every CU. The 8
//   waves of a workgroup split the k-steps of a tile; each wave keeps 5
//   k-steps (one register batch) of W in flight ahead of the MFMAs, the next
//   tile's first batch included.
//   x is staged once per workgroup into LDS as f16: row b (f32) is scaled by
//   2^sh_b (its max into [2^14, 2^15)) and split into a high part (B column
//   b) and a low part (B column 8 + b), so the products carry ~2^-22 relative
//   error; f16 x is exact in the high half alone. Rows are padded by 16 bytes,
//   which puts the 16 rows a ds_read_b128 phase touches on distinct banks.
//   The waves' 16x16 partial tiles meet in LDS (double-buffered, one barrier
//   per tile); thread (feature, b) adds the 8 waves' high and low columns,
//   scales by 2^-sh_b, adds the bias and stores.
constexpr int kGmWaves = 8;
constexpr int kGmKB = 5;          // 32-column k-steps per wave per register batch
constexpr int kGmRedPitch = 20;   // LDS pitch (floats) of one wave's 16x16 partial tile
constexpr int kGmRedFloats = 16 * kGmRedPitch;
constexpr size_t kGmStaticLds = sizeof(float) * (2 * kGmWaves * kGmRedFloats + 8);
constexpr size_t kGmMaxDynLds = 160 * 1024 - kGmStaticLds;

__device__ inline float gm_pow2(int e) { return __builtin_bit_cast(float, (e + 127) << 23); }
__device__ inline int gm_clamp_exp(int e) { return e < -126 ? -126 : (e > 127 ? 127 : e); }

__device__ inline float wave_max64(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}

template <typename XT, typename OutT, bool kLn>
__global__ __launch_bounds__(64 * kGmWaves) void gemv_f16w_mfma(GemvArgs a, int T) {
  extern __shared__ __attribute__((aligned(16))) _Float16 gxs[];  // [parts * nt][n_in + 8]
  __shared__ __attribute__((aligned(16))) float red[2][kGmWaves][kGmRedFloats];
  __shared__ float dn[8];

  constexpr bool kSplit = sizeof(XT) == 4;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 15, kg = lane >> 4;
  const int grp = blockIdx.y;
  const int nt = a.n_tokens, n_in = a.n_in, n_out = a.n_out;
  const int pitch = n_in + 8;
  const _Float16* w = a.w[grp];
  const int ks_total = n_in >> 5;
  const int s_per = (ks_total + kGmWaves - 1) / kGmWaves;
  const int ks0 = min(wave * s_per, ks_total), ks1 = min(ks0 + s_per, ks_total);
  const int n_batches = (s_per + kGmKB - 1) / kGmKB;
  const int n_tiles = (n_out + T - 1) / T;
  const bool arow = col < T;
  const u32x4 zero4 = {0, 0, 0, 0};

  // One batch of W loads; k-steps past the wave's range re-read its last
  // k-step (in bounds) and are not multiplied.
  auto load_batch = [&](int tile, int bj, u32x4 (&wv)[kGmKB]) {
    const int r = min(tile * T + (arow ? col : 0), n_out - 1);
    const _Float16* wr = w + static_cast<int64_t>(r) * n_in + 8 * kg;
#pragma unroll
    for (int u = 0; u < kGmKB; ++u) {
      const int ks = min(ks0 + bj * kGmKB + u, ks_total - 1);
      wv[u] = *reinterpret_cast<const u32x4*>(wr + 32 * ks);
    }
  };

  // f32 rows of up to 256 * kLnCache values are loaded into registers before
  // the first weight batch is issued, so that their wait does not include it
  // (loads complete in order); the arithmetic depends on a value defined after
  // both.
  int tile = blockIdx.x;
  u32x4 wv[kGmKB];
  const bool reg_row = kSplit && n_in <= 256 * kLnCache;
  f32x4 xv[kLnCache], gg[kLnCache], bb[kLnCache];
  const float* xr32 = static_cast<const float*>(a.x) + static_cast<int64_t>(wave) * a.x_rs;
  if (reg_row && wave < nt)
    ln_row_load(xr32, kLn ? a.ln_g : nullptr, a.ln_b, n_in, xv, gg, bb);
  load_batch(tile, 0, wv);  // in flight while x is staged
  float one;
  __asm__ volatile("v_mov_b32 %0, 1.0" : "=v"(one) : : "memory");

  if (reg_row && wave < nt) {
#pragma unroll
    for (int i = 0; i < kLnCache; ++i) xv[i] *= one;
    if constexpr (kLn) ln_row_norm(n_in, a.ln_eps, xv, gg, bb);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < kLnCache; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(xv[i][j]));  // zeros past n_in
    amax = wave_max64(amax);
    const int e_max = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xFF);
    const int sh = e_max == 0 ? 0 : gm_clamp_exp(141 - e_max);
    const float up = gm_pow2(sh);
#pragma unroll
    for (int i = 0; i < kLnCache; ++i) {
      const int k = 4 * lane + 256 * i;
      if (k >= n_in) break;
      f16x4v hv, lv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v = xv[i][j] * up;
        const _Float16 h = static_cast<_Float16>(v);
        hv[j] = h;
        lv[j] = static_cast<_Float16>(v - static_cast<float>(h));
      }
      *reinterpret_cast<f16x4v*>(&gxs[wave * pitch + k]) = hv;
      *reinterpret_cast<f16x4v*>(&gxs[(nt + wave) * pitch + k]) = lv;
    }
    if (lane == 0) dn[wave] = gm_pow2(gm_clamp_exp(-sh));
  }
  if constexpr (kSplit) {
    if (kLn && !reg_row && wave < nt) {
      // Longer rows with a fused LayerNorm: statistics, then two passes.
      const float* xr = xr32;
      float mean, inv_std;
      ln_row_stats(xr, n_in, a.ln_eps, mean, inv_std);
      float amax = 0.f;
      for (int k = 4 * lane; k < n_in; k += 256) {
        const f32x4 y = ln_apply(xr, a.ln_g, a.ln_b, k, mean, inv_std);
#pragma unroll
        for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(y[j]));
      }
      amax = wave_max64(amax);
      const int e_max = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xFF);
      const int sh = e_max == 0 ? 0 : gm_clamp_exp(141 - e_max);
      const float up = gm_pow2(sh);
      for (int k = 4 * lane; k < n_in; k += 256) {
        const f32x4 y = ln_apply(xr, a.ln_g, a.ln_b, k, mean, inv_std);
        f16x4v hv, lv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = y[j] * up;
          const _Float16 h = static_cast<_Float16>(v);
          hv[j] = h;
          lv[j] = static_cast<_Float16>(v - static_cast<float>(h));
        }
        *reinterpret_cast<f16x4v*>(&gxs[wave * pitch + k]) = hv;
        *reinterpret_cast<f16x4v*>(&gxs[(nt + wave) * pitch + k]) = lv;
      }
      if (lane == 0) dn[wave] = gm_pow2(gm_clamp_exp(-sh));
    }
  }
  if (wave < nt && !reg_row && !kLn) {
    const XT* xr = static_cast<const XT*>(a.x) + static_cast<int64_t>(wave) * a.x_rs;
    int sh = 0;
    if constexpr (kSplit) {
      float amax = 0.f;
      for (int k = 8 * lane; k < n_in; k += 512) {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(xr + k);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(xr + k + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fmaxf(fabsf(lo[j]), fabsf(hi[j])));
      }
      amax = wave_max64(amax);
      const int e_max = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xFF);
      sh = e_max == 0 ? 0 : gm_clamp_exp(141 - e_max);
    }
    const float up = gm_pow2(sh);
    for (int k = 8 * lane; k < n_in; k += 512) {
      f16x8 hv, lv;
      if constexpr (kSplit) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(xr + k);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(xr + k + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = (j < 4 ? x0[j] : x1[j - 4]) * up;
          const _Float16 h = static_cast<_Float16>(v);
          hv[j] = h;
          lv[j] = static_cast<_Float16>(v - static_cast<float>(h));
        }
        *reinterpret_cast<f16x8*>(&gxs[(nt + wave) * pitch + k]) = lv;
      } else {
        hv = *reinterpret_cast<const f16x8*>(xr + k);
      }
      *reinterpret_cast<f16x8*>(&gxs[wave * pitch + k]) = hv;
    }
    if (lane == 0) dn[wave] = gm_pow2(gm_clamp_exp(-sh));
  }
  __syncthreads();

  // B column c < 8: high part of x row c; c >= 8: low part of row c - 8;
  // absent rows (and the low half for f16 x) are zero.
  const int beam = col & 7;
  const bool bvalid = beam < nt && (kSplit || col < 8);
  const _Float16* xb = gxs + (bvalid ? (col < 8 ? beam : nt + beam) * pitch : 0) + 8 * kg;
  const f16x8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};

  OutT* out = reinterpret_cast<OutT*>(a.out[grp]);
  const float* bias = a.bias[grp];
  int par = 0;
  for (; tile < n_tiles; tile += gridDim.x) {
    // Bias of the feature this thread stores, loaded under the MFMAs.
    float bias_v = 0.f;
    if (bias && tid < 128) bias_v = bias[min(tile * T + min(tid >> 3, T - 1), n_out - 1)];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int bj = 0; bj < n_batches; ++bj) {
      u32x4 cur[kGmKB];
#pragma unroll
      for (int u = 0; u < kGmKB; ++u) cur[u] = arow ? wv[u] : zero4;
      if (bj + 1 < n_batches)
        load_batch(tile, bj + 1, wv);
      else if (tile + static_cast<int>(gridDim.x) < n_tiles)
        load_batch(tile + gridDim.x, 0, wv);
#pragma unroll
      for (int u = 0; u < kGmKB; ++u) {
        const int ks = ks0 + bj * kGmKB + u;
        if (ks < ks1) {  // wave-uniform
          const f16x8 bx = bvalid ? *reinterpret_cast<const f16x8*>(xb + 32 * ks) : zero8;
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, cur[u]), bx, acc,
                                                       0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[par][wave][(4 * kg + i) * kGmRedPitch + col] = acc[i];
    __syncthreads();
    if (tid < 128) {
      const int r = tid >> 3, b = tid & 7;
      const int row = tile * T + r;
      if (r < T && b < nt && row < n_out) {
        float sacc = 0.f;
#pragma unroll
        for (int w8 = 0; w8 < kGmWaves; ++w8)
          sacc += red[par][w8][r * kGmRedPitch + b] + red[par][w8][r * kGmRedPitch + b + 8];
        float v = sacc * dn[b];
        if (bias) v += bias_v;
        if (a.act == kActGelu) v = gelu_tanh(v);
        out[static_cast<int64_t>(b) * a.out_rs + static_cast<int64_t>(row >> 6) * a.out_hs +
            (row & 63)] = static_cast<OutT>(v);
      }
    }
    par ^= 1;
  }
}

// f32 rows -> [hi | lo] f16 rows of 2 n_in, plus each row's 2^-shift.
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
  _Float16* dst = xs + static_cast<int64_t>(t) * kSplitParts * n_in;
  for (int k = lane; k < n_in; k += 64) {
    const float v = xr[k] * up;
    const _Float16 h = static_cast<_Float16>(v);
    dst[k] = h;
    dst[n_in + k] = static_cast<_Float16>(v - static_cast<float>(h));
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

hipError_t launch_gemv_f16w(const GemvArgs& a, DType x_dt, DType out_dt, hipStream_t s) {
  if (a.n_tokens <= 0 || a.n_out <= 0 || a.n_groups <= 0) return hipSuccess;
  if (a.n_tokens > kGemvMaxRows) return hipErrorInvalidValue;
  if (a.n_tokens * a.n_in > kGemvXFloats) return hipErrorInvalidValue;
  int dev = 0, n_cu = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  // Three or more x rows: the matrix-pipe kernel (one or two rows read the
  // staged x cheaply enough that the FMA kernel's wider spread wins).
  const size_t gm_lds = static_cast<size_t>(x_dt == kF32 ? 2 : 1) * a.n_tokens * (a.n_in + 8) * 2;
  if (a.n_tokens >= 3 && (a.n_in & 31) == 0 && gm_lds <= kGmMaxDynLds &&
      (x_dt == kF32 || x_dt == kF16)) {
    // Tiles of T features, T chosen so that the tiles of all groups just
    // cover one workgroup per CU (a d x d matrix measured fastest that way:
    // two smaller tiles per CU stage x twice), or exactly k per CU when one
    // per CU would need more than 16 features: a 5120-row matrix in 16-feature
    // tiles gave 64 CUs two tiles and the rest one. Up to as many workgroups
    // as fit at once (LDS and registers decide) share the tiles, looping.
    const dim3 gblock(64 * kGmWaves);
#define WRS_GM_L(XT, OT, LN)                                                                  \
  {                                                                                           \
    const void* fn = reinterpret_cast<const void*>(&gemv_f16w_mfma<XT, OT, LN>);              \
    static std::atomic<uint64_t> attr_set{0};  /* one bit per device */                       \
    if (dev < 64 && !(attr_set.load(std::memory_order_acquire) & (uint64_t{1} << dev))) {     \
      const hipError_t e = hipFuncSetAttribute(                                               \
          fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kGmMaxDynLds));    \
      if (e != hipSuccess) return e;                                                          \
      attr_set.fetch_or(uint64_t{1} << dev, std::memory_order_acq_rel);                       \
    }                                                                                         \
    int per_cu = 1;                                                                           \
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, gblock.x, gm_lds) !=         \
            hipSuccess ||                                                                     \
        per_cu < 1)                                                                           \
      per_cu = 1;                                                                             \
    const int64_t rows = static_cast<int64_t>(a.n_out) * a.n_groups;                         \
    const int64_t per_cu_tiles = (rows + 16 * n_cu - 1) / (16 * n_cu);                      \
    const int T = static_cast<int>(std::max<int64_t>(                                        \
        1, std::min<int64_t>(16, (rows + per_cu_tiles * n_cu - 1) / (per_cu_tiles * n_cu)))); \
    const int n_tiles = (a.n_out + T - 1) / T;                                                \
    const dim3 ggrid(std::min(n_tiles, n_cu * std::min(per_cu, 2)), a.n_groups);              \
    hipLaunchKernelGGL((gemv_f16w_mfma<XT, OT, LN>), ggrid, gblock, gm_lds, s, a, T);         \
  }
#define WRS_GM(XT, OT)                 \
  if (a.ln_g) {                        \
    WRS_GM_L(XT, OT, true)             \
  } else {                             \
    WRS_GM_L(XT, OT, false)            \
  }
#define WRS_GM16(XT, OT) WRS_GM_L(XT, OT, false)
    if (x_dt == kF32) {
      switch (out_dt) {
        case kF32: WRS_GM(float, float); break;
        case kF16: WRS_GM(float, _Float16); break;
        case kBF16: WRS_GM(float, __bf16); break;
        default: return hipErrorInvalidValue;
      }
    } else {
      if (a.ln_g) return hipErrorInvalidValue;  // the fused LayerNorm takes f32 rows
      switch (out_dt) {
        case kF32: WRS_GM16(_Float16, float); break;
        case kF16: WRS_GM16(_Float16, _Float16); break;
        case kBF16: WRS_GM16(_Float16, __bf16); break;
        default: return hipErrorInvalidValue;
      }
    }
#undef WRS_GM16
#undef WRS_GM
#undef WRS_GM_L
    return hipGetLastError();
  }
  // Up to kGemvSmallOut features: one feature per wave, so that the matrix
  // spreads over ~n_out / 8 CUs; beyond it 4 features per wave share each
  // staged x read.
  const int rpw = a.n_out <= kGemvSmallOut ? 1 : 4;
  const int groups = (a.n_out + rpw - 1) / rpw;
  const int wgs = std::min(n_cu, (groups + kGemvWaves - 1) / kGemvWaves);
  dim3 grid(std::max(wgs, 1), a.n_groups);
  dim3 block(64 * kGemvWaves);
#define WRS_GEMV_R(R, XT, OT)                                                           \
  switch (a.n_tokens) {                                                                 \
    case 1: hipLaunchKernelGGL((gemv_f16w<1, R, XT, OT>), grid, block, 0, s, a); break;  \
    case 2: hipLaunchKernelGGL((gemv_f16w<2, R, XT, OT>), grid, block, 0, s, a); break;  \
    case 3: hipLaunchKernelGGL((gemv_f16w<3, R, XT, OT>), grid, block, 0, s, a); break;  \
    case 4: hipLaunchKernelGGL((gemv_f16w<4, R, XT, OT>), grid, block, 0, s, a); break;  \
    case 5: hipLaunchKernelGGL((gemv_f16w<5, R, XT, OT>), grid, block, 0, s, a); break;  \
    case 6: hipLaunchKernelGGL((gemv_f16w<6, R, XT, OT>), grid, block, 0, s, a); break;  \
    case 7: hipLaunchKernelGGL((gemv_f16w<7, R, XT, OT>), grid, block, 0, s, a); break;  \
    default: hipLaunchKernelGGL((gemv_f16w<8, R, XT, OT>), grid, block, 0, s, a); break; \
  }
#define WRS_GEMV(XT, OT)          \
  if (rpw == 1) {                 \
    WRS_GEMV_R(1, XT, OT)         \
  } else {                        \
    WRS_GEMV_R(4, XT, OT)         \
  }
  if (x_dt == kF32) {
    switch (out_dt) {
      case kF32: WRS_GEMV(float, float); break;
      case kF16: WRS_GEMV(float, _Float16); break;
      case kBF16: WRS_GEMV(float, __bf16); break;
      default: return hipErrorInvalidValue;
    }
  } else if (x_dt == kF16) {
    switch (out_dt) {
      case kF32: WRS_GEMV(_Float16, float); break;
      case kF16: WRS_GEMV(_Float16, _Float16); break;
      case kBF16: WRS_GEMV(_Float16, __bf16); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
#undef WRS_GEMV
#undef WRS_GEMV_R
  return hipGetLastError();
}

hipError_t launch_linear_f16w(const LinearArgs& a, DType out_dt, hipStream_t s) {
  if (a.n_tokens <= 0 || a.n_out <= 0 || a.n_groups <= 0) return hipSuccess;
  dim3 grid(((a.n_out + kBM - 1) / kBM) * ((a.n_tokens + kBN - 1) / kBN), 1, a.n_groups);
  switch (out_dt) {
    case kF32: hipLaunchKernelGGL(linear_f16w<float>, grid, dim3(kThreads), 0, s, a); break;
    case kF16: hipLaunchKernelGGL(linear_f16w<_Float16>, grid, dim3(kThreads), 0, s, a); break;
    case kBF16: hipLaunchKernelGGL(linear_f16w<__bf16>, grid, dim3(kThreads), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace wrs
