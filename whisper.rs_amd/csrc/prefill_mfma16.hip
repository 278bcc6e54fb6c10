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
// (window, head), two workgroups per CU; each wave owns two 32-query blocks.
// Smaller grids take 128-query workgroups (one block per wave), 8-wave ones
// whose halves split the keys, or the key split (K1s, below);
// launch_prefill_mfma16 picks by grid size.
// Computing S^T = K Q^T (keys on the MFMA M axis) puts one query per lane, and
// the S^T accumulator registers are, after exp2 and packing, exactly the B
// operand of O^T += V^T P^T. Every K and V^T operand read from LDS feeds the
// MFMAs of both query blocks. V stays row-major in LDS; the transposed A
// operand of the PV product comes from ds_read_b64_tr_b16.
//
// Per 32-key step j a wave issues, as one basic block, the S^T MFMAs of step
// j+1 and the PV MFMAs of step j-1 interleaved with the softmax weights of
// step j (VALU), then the row sums of step j (16x16x32 MFMAs with a 0/1
// selector operand, which keeps the sum off the VALU) and the LDS operand
// reads for the next step. At d_head 64 the softmax VALU work is the bound,
// so it carries nothing the matrix pipe can do.
//
// K/V tiles (64 keys) move from global memory straight into LDS with
// buffer_load ... lds (no staging registers); rows past t_kv read as zero
// through the buffer range check. Tiles are stored unpadded with the 16-byte
// chunks of each 128-byte row XOR-swizzled, so both the K operand reads (rows
// r..r+15, one chunk) and the transposed V reads (rows 4i..4i+3, a chunk pair)
// are free of bank conflicts. Four tile buffers: the steps of tile t read
// tiles t and t+1, tile t+2 lands, tile t+3 is issued; one barrier per tile.
// For bf16 inputs each wave converts its own V rows to f16 in place once they
// land (exact in the f16 normal range).
//
// Softmax rescaling is lazy: weights are formed against a reference max that
// may lag the true row max. A step is checked when some query's row sum over
// it exceeds 2^14 (which bounds every weight inside the f16 range) or twice
// the query's row sum over all earlier steps. Then every query whose step max
// lies above its reference moves the reference there (scaling O and l), and,
// if any did, the step's weights are formed again. The second condition puts
// the reference on the dominant key of a peaked row, whose weight is then
// exactly 1 instead of an f16-rounded value up to 2^14: with rounded dominant
// weights the error reaches 2^-12 of the V range, with exact ones it stays
// near the diffuse rows' level. A diffuse row rarely has one step outweigh all
// earlier ones, so the weights are formed again on about 5% of steps. The
// first step takes its reference max from the (masked) scores of the first
// two steps before forming its weights, so neither forms them twice.
#include "prefill_f32_block.hpp"
#include "wrs_internal.hpp"

#include <type_traits>

namespace wrs {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kN = 64;              // keys per tile
constexpr int kNB = 4;              // LDS tile buffers
constexpr int kTileH = kN * 64;     // 16-bit elements per K (or V) tile: 8 KiB
constexpr int kRowsPerWave = kN / kWaves;  // tile rows one wave copies
constexpr int kRowGroups = kRowsPerWave / 8;  // one 1 KiB DMA per 8 rows
constexpr int kDmaPerTile = 2 * kRowGroups;   // K and V
// Split blocks: floats one wave publishes (its 16 O registers, max and sum,
// each for 64 lanes), and words between merge counters (one 128-byte line
// each).
constexpr int kSplitPartWave = 18 * 64;
constexpr int kSplitCounterStride = 32;
constexpr int kSplitPartWg = 2 * kWaves * kSplitPartWave;  // one split workgroup's partial
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kSumLimit = 16384.0f;  // row sum of one step that forces a rescale
constexpr float kNoMax = -1.0e30f;     // reference max before the first step

template <typename T>
struct Elem;

template <>
struct Elem<_Float16> {
  static constexpr bool kConvertV = false;
  static __device__ inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ inline u32x4 to_f16(u32x4 x) { return x; }
};

template <>
struct Elem<__bf16> {
  static constexpr bool kConvertV = true;
  static __device__ inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // bf16 -> f16: widening to f32 is a shift and the f32 -> f16 rounding is
  // exact for bf16 values inside the f16 normal range.
  static __device__ inline u32x4 to_f16(u32x4 x) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t xi = x[i];
      const f32x2 w = {__builtin_bit_cast(float, xi << 16),
                       __builtin_bit_cast(float, xi & 0xffff0000u)};
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

// Four consecutive keys of one d column of a row-major [key][d] LDS tile, from
// an LDS byte address; and 16 bytes at one.
__device__ inline u32x2 read_tr_at(uint32_t addr) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)addr);
  return __builtin_bit_cast(u32x2, v);
}
__device__ inline u32x4 lds_read16(uint32_t addr) {
  return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)addr;
}

// 16-byte chunk swizzle of a 128-byte tile row: chunk c of row r is stored at
// c ^ swz(r). Sixteen consecutive rows reading one chunk, and four rows
// 4i..4i+3 reading an aligned chunk pair, then hit distinct banks.
__device__ inline int swz(int r) {
  return ((2 * (r & 3)) | ((r >> 2) & 1)) ^ (((r >> 3) & 1) << 1);
}

// 16 bytes per lane from global memory into LDS at m0 + 16 * lane, through a
// buffer resource (out-of-range offsets read as zero). Issued as inline asm so
// that the compiler adds no waits of its own before later LDS reads: the
// caller orders it with explicit vmcnt waits and barriers. m0 is written here
// and used by nothing else in this kernel.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
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

// This wave's LDS traffic is complete, then all waves meet (no vmcnt wait:
// tile loads in flight stay in flight).
__device__ inline void tile_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
// Wait until at most N of this wave's tile loads are in flight.
template <int N>
__device__ inline void wait_tiles() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// QB: 32-query blocks per wave (2, or 1 for grids below one round of
// workgroups); QW: waves that share a workgroup's queries (4, or 6); a
// workgroup holds 32 * QB * QW queries.
template <int QB, int QW = kWaves>
constexpr int queries_per_wg() {
  return 32 * QB * QW;
}

// Software pipeline of a full 32-key step (see full_step in the kernel): one
// big MFMA per slot, 8*QB slots; unit u (two scores of block u/8, one packed
// f16 register) has its FMAs in slot pipe_fma_slot(u), exp2 in the next slot
// and the pack in the one after; block jb's row sums follow its last pack.
template <int QB>
constexpr int kSlots() {
  return 8 * QB;
}
constexpr int pipe_fma_slot(int u) { return (2 * u) / 3; }
constexpr int pipe_rowsum_slot(int jb) { return pipe_fma_slot(8 * jb + 7) + 3; }
// Program order must respect the data flow: the pack of unit u overwrites
// register pb[u/8][(u/4)%2] after the P V MFMAs of the previous step have read
// it (slots 4*jb + 2*k2 + {0, 1}), and every pack and row sum falls inside the
// step.
template <int QB>
constexpr bool pipe_order_ok() {
  for (int u = 0; u < 8 * QB; ++u) {
    const int jb = u >> 3, k2 = (u >> 2) & 1;
    if (pipe_fma_slot(u) + 2 < 4 * jb + 2 * k2 + 1) return false;
    if (pipe_fma_slot(u) + 2 >= kSlots<QB>()) return false;
  }
  for (int jb = 0; jb < QB; ++jb)
    if (pipe_rowsum_slot(jb) >= kSlots<QB>()) return false;
  return true;
}
static_assert(pipe_order_ok<1>() && pipe_order_ok<2>(), "pipelined step order");

// KH = 2 (key halves): the workgroup is two halves of QW waves that share its
// 32 * QB * QW queries and split its keys, half hf taking the 64-key tiles
// hf, hf + 2, ... through its own LDS ring; the halves then merge their
// (max, sum, O) lane by lane (their registers hold the same queries in the
// same layout). For grids of at most one such workgroup per CU, it puts two
// waves (three with QW = 6) on every SIMD of the CUs in use instead of one.
// With QW = 6 the first four waves of a half move its tiles and the other
// two only compute. WS > 1 (split blocks): a block's keys are shared by WS
// such workgroups, its tiles falling into KH * WS parts taken in turn, and
// the workgroups merge through memory.
template <typename T, int QB, int KH, int QW = kWaves, int WS = 1>
__global__ __launch_bounds__(64 * QW * KH, 2 / KH) void fa2_prefill_d64(
    PrefillArgs a, int n_qblk) {
  static_assert(KH == 1 || KH == 2, "one or two key halves");
  static_assert(WS == 1 || ((WS == 2 || WS == 3) && KH == 2 && QB == 1 && QW == kWaves),
                "blocks split over two or three workgroups: 128 queries, key halves");
  static_assert(QW == kWaves || (QW == 6 && QB == 1 && KH == 2),
                "six query waves: one block each, key halves");
  constexpr int kQB = QB;
  constexpr int kM = queries_per_wg<QB, QW>();
  typedef f32x16 SBlk[kQB];
  typedef u32x4 PBlk[kQB][2];
  __shared__ __attribute__((aligned(128))) uint16_t Ks[KH * kNB * kTileH];
  __shared__ __attribute__((aligned(128))) uint16_t Vs[KH * kNB * kTileH];
  __shared__ int nonfinite;  // bf16: some output of the workgroup is inf/NaN
  __shared__ int merger;     // split blocks: this workgroup merges the block
  static_assert(sizeof(f32blk::Tiles<2>) <= sizeof(Ks), "f32 tiles fit in the K buffers");

  const int lid = __builtin_amdgcn_readfirstlane(xcd_remap(blockIdx.x, gridDim.x));
  // Split blocks: the block's WS workgroups are neighbours in lid (one XCD).
  const int wsplit = WS == 1 ? 0 : lid % WS;
  const int blk = WS == 1 ? lid : lid / WS;  // (window, head, query block)
  const int qblk = blk % n_qblk;
  const int bh = blk / n_qblk;
  const int h = bh % a.n_heads;
  const int b = bh / a.n_heads;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hl = lane >> 5;
  // Key half of this wave, its place among the half's waves, and the half's
  // tile ring.
  const int half = KH == 1 ? 0 : QW == kWaves ? (wave >> 2) : wave / QW;
  const int wq = KH == 1 ? wave : QW == kWaves ? (wave & 3) : wave - QW * half;
  // The first four waves of a half move its tiles (16 rows of each apiece).
  const bool mover = QW == kWaves || wq < kWaves;
  uint16_t* const Kh = Ks + half * (kNB * kTileH);
  uint16_t* const Vh = Vs + half * (kNB * kTileH);
  // Cleared before the first tile barrier; set only after the last one.
  if (tid == 0) nonfinite = 0;

  const T* qp = static_cast<const T*>(a.q) + b * a.lq.bs + h * a.lq.hs;
  const T* kp = static_cast<const T*>(a.k) + b * a.lk.bs + h * a.lk.hs;
  const T* vp = static_cast<const T*>(a.v) + b * a.lv.bs + h * a.lv.hs;

  // This lane's queries: column r32 of each of the wave's S^T blocks.
  const int q0 = qblk * kM + wq * (32 * kQB) + r32;
  u32x4 qf[kQB][4];
#pragma unroll
  for (int j = 0; j < kQB; ++j) {
    if (q0 + 32 * j < a.t_q) {
      const T* row = qp + static_cast<int64_t>(q0 + 32 * j) * a.lq.rs + hl * 8;
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
  const int n_tiles_all = (kv_end + kN - 1) / kN;
  // The block's tiles fall into kP parts taken in turn (key halves, over WS
  // workgroups): this half's part, its tiles (local tile t is tile kP t + part
  // of the block's keys) and the most that a half of this workgroup has.
  constexpr int kP = KH * WS;
  const int part = KH * wsplit + half;
  const int n_tiles = (n_tiles_all - part + kP - 1) / kP;
  const int t_most = (n_tiles_all - KH * wsplit + kP - 1) / kP;
  const int nh = 2 * n_tiles;  // this half's 32-key steps
  // The block's 32-key step of this half's step j.
  auto gstep = [&](int j) { return 2 * (kP * (j >> 1) + part) + (j & 1); };
  // First step that needs a mask: keys past t_kv, or (causal) past the first
  // query of the workgroup.
  int first_masked = a.t_kv / 32;
  if (a.causal) first_masked = min(first_masked, (qblk * kM + a.q_pos_offset + 1) / 32);

  // Tile copy: wave w moves rows kRowsPerWave*w.. of each K and V tile, 8
  // rows (1 KiB, one DMA) at a time; lane i carries row i/8, chunk i%8 of them.
  uint32_t kofs[kRowGroups], vofs[kRowGroups];
#pragma unroll
  for (int r = 0; r < kRowGroups; ++r) {
    const int crow = kRowsPerWave * wq + 8 * r + (lane >> 3);
    const int cch = (lane & 7) ^ swz(crow);
    kofs[r] = static_cast<uint32_t>((crow * a.lk.rs + cch * 8) * 2);
    vofs[r] = static_cast<uint32_t>((crow * a.lv.rs + cch * 8) * 2);
  }
  const uint32_t kstep = static_cast<uint32_t>(kN * a.lk.rs * 2);
  const uint32_t vstep = static_cast<uint32_t>(kN * a.lv.rs * 2);
  const u32x4 krs = buffer_rsrc(kp, static_cast<uint32_t>(((a.t_kv - 1) * a.lk.rs + 64) * 2));
  const u32x4 vrs = buffer_rsrc(vp, static_cast<uint32_t>(((a.t_kv - 1) * a.lv.rs + 64) * 2));
  const uint32_t ks_lds = lds_addr(Kh) + wq * kRowsPerWave * 128;
  const uint32_t vs_lds = lds_addr(Vh) + wq * kRowsPerWave * 128;
  auto issue_tile = [&](int t) {
    if (!mover) return;
    const uint32_t buf = __builtin_amdgcn_readfirstlane((t % kNB) * (kTileH * 2));
#pragma unroll
    for (int r = 0; r < kRowGroups; ++r)
      dma16(krs, ks_lds + buf + 1024 * r, kofs[r] + (kP * t + part) * kstep);
#pragma unroll
    for (int r = 0; r < kRowGroups; ++r)
      dma16(vrs, vs_lds + buf + 1024 * r, vofs[r] + (kP * t + part) * vstep);
  };
  // bf16 V -> f16 in place: this wave's own rows, whose loads have landed.
  auto convert_tile = [&](int t) {
    if constexpr (Elem<T>::kConvertV) {
      if (!mover) return;
#pragma unroll
      for (int r = 0; r < kRowGroups; ++r) {
        u32x4* p = reinterpret_cast<u32x4*>(Vh + (t % kNB) * kTileH + wq * kRowsPerWave * 64 +
                                            r * 512 + lane * 8);
        *p = Elem<T>::to_f16(*p);
      }
    }
  };

  // Per-lane LDS byte offsets of the MFMA operand reads, as one base per
  // operand and XOR masks. K A operand: row r32, 16-byte chunk
  // (hl + 2*dk) ^ swz(r32) = (hl ^ swz(r32)) ^ 2*dk, i.e. the base XOR 32*dk.
  // V^T operand (transposed read): lane group g = lane/16 reads rows
  // r0 = 4*(g/2) + (lane%16)/4 [+8*e] at columns 16*(g%2) + 4*(lane%4)
  // [+32*cc], so lane (d, hl) receives keys 4*hl + 0..3 [+8]. Row r0 + 8 has
  // swz(r0) ^ 2, and chunk c0 + 4 = c0 ^ 4, so operand (e, cc) sits at the
  // base + 1024*e, XOR 64*cc + 32*e. The masks touch bits 5-6 only and the
  // tile buffers are 128-byte aligned, so they apply to whole LDS addresses.
  const uint32_t koff0 = static_cast<uint32_t>(r32 * 128 + ((hl ^ swz(r32)) * 16));
  const int g = lane >> 4, t4 = lane & 15;
  const int vr0 = 4 * (g >> 1) + (t4 >> 2), vc0 = 2 * (g & 1) + ((t4 & 3) >> 1);
  const uint32_t voff0 = static_cast<uint32_t>(vr0 * 128 + ((vc0 ^ swz(vr0)) * 16) + 8 * (t4 & 1));
  auto k_base = [&](int step) {
    return lds_addr(Kh) + ((step >> 1) % kNB) * (kTileH * 2) + (step & 1) * 32 * 128 + koff0;
  };
  auto kfetch = [&](int step, u32x4 (&ka)[4]) {
    const uint32_t kb = k_base(step);
#pragma unroll
    for (int dk = 0; dk < 4; ++dk) ka[dk] = lds_read16(kb ^ (32u * dk));
  };
  auto vfetch = [&](int step, u32x2 (&va)[8]) {
    const uint32_t vb =
        lds_addr(Vh) + ((step >> 1) % kNB) * (kTileH * 2) + (step & 1) * 32 * 128 + voff0;
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const uint32_t x = (vb ^ (64u * cc + 32u * e)) + 1024u * e;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) va[4 * k2 + 2 * cc + e] = read_tr_at(x + 2048u * k2);
      }
  };
  // S^T = K Q^T for 32 keys and both query blocks.
  auto qk = [&](const u32x4 (&ka)[4], SBlk& s) {
#pragma unroll
    for (int j = 0; j < kQB; ++j) s[j] = f32x16{};
#pragma unroll
    for (int dk = 0; dk < 4; ++dk)
#pragma unroll
      for (int j = 0; j < kQB; ++j) s[j] = Elem<T>::mfma(ka[dk], qf[j][dk], s[j]);
  };

  const float c = a.scale * kLog2e;  // exp(scale*s - m') == exp2(c*s - m)
  f32x16 o[kQB][2];                  // O^T rows d 0..31 / 32..63, column = query
  float m[kQB], l[kQB];              // reference max (exp2 domain), partial row sum
#pragma unroll
  for (int j = 0; j < kQB; ++j) {
    o[j][0] = o[j][1] = f32x16{};
    m[j] = kNoMax;
    l[j] = 0.f;
  }

  // Accumulator register i of a 32x32 block holds key 8*(i/4) + 4*hl + i%4 of
  // its 32-key step.
  auto mask_step = [&](int step, SBlk& s) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kr = 32 * step + 8 * (i >> 2) + 4 * hl + (i & 3);
#pragma unroll
      for (int j = 0; j < kQB; ++j) {
        const int qpos = q0 + 32 * j + a.q_pos_offset;
        s[j][i] = ((kr >= a.t_kv) | ((a.causal != 0) & (kr > qpos))) ? -INFINITY : s[j][i];
      }
    }
  };
  // P = exp2(c*S - m) as packed f16 pairs, already in B-operand order for the
  // PV product: block k2 covers step keys 16*k2 + 8*(w/2) + 4*hl + {0..3}.
  auto weights = [&](const SBlk& s, PBlk& pb) {
#pragma unroll
    for (int j = 0; j < kQB; ++j)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const f32x2 pp = {
              __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][8 * k2 + 2 * w], c, -m[j])),
              __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][8 * k2 + 2 * w + 1], c, -m[j]))};
          pb[j][k2][w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pp, f16x2));
        }
  };
  // Row sums of the rounded weights on the matrix pipe. Read as the B operand
  // of a 16x16x32 MFMA, the weight registers of 16 keys put the keys of query
  // n (lanes n and n+32, n < 32) in column n mod 16, k-groups n/16 and n/16+2.
  // A selector A operand that is 1 exactly where (row/4) and the k-group have
  // the same parity leaves, in every register of lane l, the f32 sum of the
  // 16 weights of query l mod 32. Rows of the other query in the column meet
  // zeros, so an infinite weight there turns this sum into NaN; the rescale
  // check below treats NaN like an overflow.
  const _Float16 rs_one = ((lane >> 2) & 1) == ((lane >> 4) & 1) ? 1.0f16 : 0.0f16;
  const f16x8 rs_sel = {rs_one, rs_one, rs_one, rs_one, rs_one, rs_one, rs_one, rs_one};
  auto row_sums = [&](const PBlk& pb, f32x4 (&ls)[kQB]) {
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      const f32x4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          rs_sel, __builtin_bit_cast(f16x8, pb[j][0]), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      ls[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(rs_sel, __builtin_bit_cast(f16x8, pb[j][1]),
                                                     acc, 0, 0, 0);
    }
  };
  // O^T += V^T P^T for one 32-key step.
  auto pv = [&](const u32x2 (&va)[8], const PBlk& pb) {
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
  // Lazy rescale (see the file header): after a step's weights are formed,
  // move the reference max when some lane's partial row sum is out of range
  // (the first step has already taken its max), rescale O and l, and form the weights again;
  // then fold the step's row sums into l.
  // Does some query of the wave need its reference max checked? Unsigned
  // compares of the bit patterns: true for sums above the limit or above the
  // earlier steps' sum, inf and NaN alike (the kernel is built without NaN
  // semantics, so a float compare may not see NaN). Row sums are never
  // negative; 2 * l is l plus one in its exponent field (l is finite, and 0
  // before the first step).
  auto needs_check = [&](const f32x4 (&ls)[kQB]) {
    bool need = false;
#pragma unroll
    for (int j = 0; j < kQB; ++j)
      need |= __builtin_bit_cast(uint32_t, ls[j][0]) >
              min(__builtin_bit_cast(uint32_t, l[j]) + 0x00800000u,
                  __builtin_bit_cast(uint32_t, kSumLimit));
    return __builtin_amdgcn_ballot_w64(need) != 0;
  };
  // Move the reference max of every query whose step max lies above it
  // (scaling O and l), and form the step's weights again if any query moved.
  auto move_max = [&](const SBlk& s, PBlk& pb, f32x4 (&ls)[kQB]) {
    bool moved = false;
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      float mr = fmaxf(s[j][0], s[j][1]);
#pragma unroll
      for (int i = 2; i < 16; i += 2) mr = fmaxf(fmaxf(mr, s[j][i]), s[j][i + 1]);  // v_max3
      const float mx = pair_max(mr) * c;
      if (mx > m[j]) {
        const float alpha = __builtin_amdgcn_exp2f(m[j] - mx);
        m[j] = mx;
        l[j] *= alpha;
        o[j][0] *= alpha;
        o[j][1] *= alpha;
        moved = true;
      }
    }
    if (__builtin_amdgcn_ballot_w64(moved)) {
      weights(s, pb);
      row_sums(pb, ls);
    }
  };
  auto settle = [&](const SBlk& s, PBlk& pb, f32x4 (&ls)[kQB]) {
    if (needs_check(ls)) move_max(s, pb, ls);
#pragma unroll
    for (int j = 0; j < kQB; ++j) l[j] += ls[j][0];
  };

  if (n_tiles > 0) {
    issue_tile(0);
    if (n_tiles > 1) issue_tile(1);
    if (n_tiles > 2) issue_tile(2);
    wait_tiles<0>();
    convert_tile(0);
    if (n_tiles > 1) convert_tile(1);
    if (n_tiles > 2) convert_tile(2);
    tile_barrier();

    SBlk sa, sb;
    PBlk pb;
    u32x4 ka[4];
    u32x2 va[8];
    f32x4 ls[kQB];
    kfetch(0, ka);
    qk(ka, sa);
    kfetch(1, ka);

    // Step j: S of step j+1, weights and row sums of step j, PV of step j-1,
    // then the operand reads for the next step (K of step j+2, V of step j),
    // then the lazy-rescale check of step j. This form serves the first step
    // and the masked tail; full steps (every part present, no mask) take the
    // pipelined form below.
    auto part_step = [&](int j, SBlk& s_in, SBlk& s_out) __attribute__((always_inline)) {
      // P V of step j-1 first: its weights' registers are then free for step j's.
      if (j >= 1) pv(va, pb);
      if (j + 1 < nh) qk(ka, s_out);
      if (gstep(j) >= first_masked) mask_step(gstep(j), s_in);
      if (j == 0) {
        // First step: take the reference max from the (masked) scores of the
        // first two steps now (those of step 1 were just issued above), so the
        // weights of both are formed against their exact max and once.
        const bool two = nh > 1;
        if (two && gstep(1) >= first_masked) mask_step(gstep(1), s_out);
#pragma unroll
        for (int jb = 0; jb < kQB; ++jb) {
          float mr = fmaxf(s_in[jb][0], s_in[jb][1]);
#pragma unroll
          for (int i = 2; i < 16; i += 2) mr = fmaxf(fmaxf(mr, s_in[jb][i]), s_in[jb][i + 1]);
          if (two) {
#pragma unroll
            for (int i = 0; i < 16; i += 2) mr = fmaxf(fmaxf(mr, s_out[jb][i]), s_out[jb][i + 1]);
          }
          const float mx = pair_max(mr) * c;
          if (mx > m[jb]) m[jb] = mx;
        }
      }
      weights(s_in, pb);
      row_sums(pb, ls);
      if (j + 2 < nh) kfetch(j + 2, ka);
      vfetch(j, va);
      __builtin_amdgcn_sched_barrier(0);
      settle(s_in, pb, ls);
      __builtin_amdgcn_sched_barrier(0);
    };

    // Full step j, software-pipelined. Slot n (0 <= n < 8*QB) issues one
    // 32x32x16 MFMA -- P V of step j-1 for n < 4*QB, S of step j+1 after --
    // and then the VALU work assigned to it. The weights of step j form in
    // 8*QB units of two scores (one packed f16 register): unit u's FMAs run in
    // slot pipe_fma_slot(u), its exp2 one slot later and its pack one slot
    // after that, so no instruction waits on the result of the one before it
    // (as a chain FMA -> exp2 -> pack through two temporaries would, on the
    // exp2 latency, with the matrix pipe idle meanwhile). S of step j is
    // overwritten in place: its registers hold the weights in f32 until they
    // are packed. The rare rescale path computes S again from the K tile,
    // still in LDS, with the same MFMAs in the same order (bit for bit the
    // same scores). A sched_barrier ends each slot, so its instructions stay
    // together.
    auto full_step = [&](int j, SBlk& s, SBlk& s_next) __attribute__((always_inline)) {
      const uint32_t kb2 = k_base(j + 2);
#pragma unroll
      for (int n = 0; n < kSlots<kQB>(); ++n) {
        if (n < 4 * kQB) {
          const int jb = n >> 2, k2 = (n >> 1) & 1, hf = n & 1;
          const u32x2 v0 = va[4 * k2 + 2 * hf], v1 = va[4 * k2 + 2 * hf + 1];
          o[jb][hf] = mfma_f16(u32x4{v0.x, v0.y, v1.x, v1.y}, pb[jb][k2], o[jb][hf]);
        } else {
          const int qn = n - 4 * kQB;
          const int dk = qn / kQB, jb = qn % kQB;
          s_next[jb] = Elem<T>::mfma(ka[dk], qf[jb][dk], dk == 0 ? f32x16{} : s_next[jb]);
        }
#pragma unroll
        for (int u = 0; u < 8 * kQB; ++u) {
          const int jb = u >> 3, k2 = (u >> 2) & 1, w = u & 3, i = 8 * k2 + 2 * w;
          if (pipe_fma_slot(u) + 2 == n) {
            const f32x2 pp = {s[jb][i], s[jb][i + 1]};
            pb[jb][k2][w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pp, f16x2));
          }
          if (pipe_fma_slot(u) + 1 == n) {
            s[jb][i] = __builtin_amdgcn_exp2f(s[jb][i]);
            s[jb][i + 1] = __builtin_amdgcn_exp2f(s[jb][i + 1]);
          }
          if (pipe_fma_slot(u) == n) {
            s[jb][i] = __builtin_fmaf(s[jb][i], c, -m[jb]);
            s[jb][i + 1] = __builtin_fmaf(s[jb][i + 1], c, -m[jb]);
          }
        }
#pragma unroll
        for (int jb = 0; jb < kQB; ++jb) {
          if (pipe_rowsum_slot(jb) == n) {
            const f32x4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                rs_sel, __builtin_bit_cast(f16x8, pb[jb][0]), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            ls[jb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                rs_sel, __builtin_bit_cast(f16x8, pb[jb][1]), acc, 0, 0, 0);
          }
        }
        // Operand reads for later steps, each after the last MFMA that reads
        // the registers it fills: V of step j once P V is issued, K of step
        // j+2 chunk by chunk behind the S MFMAs.
        if (n == 4 * kQB) vfetch(j, va);
#pragma unroll
        for (int dk = 0; dk < 3; ++dk)
          if (n == 4 * kQB + (dk + 1) * kQB)
            ka[dk] = lds_read16(kb2 ^ (32u * dk));
        __builtin_amdgcn_sched_barrier(0);
      }
      ka[3] = lds_read16(kb2 ^ 96u);
      if (needs_check(ls)) {
        // K of step j into the operand registers, then K of step j+2 again.
        kfetch(j, ka);
        qk(ka, s);
        kfetch(j + 2, ka);
        move_max(s, pb, ls);
      }
#pragma unroll
      for (int jb = 0; jb < kQB; ++jb) l[jb] += ls[jb][0];
      __builtin_amdgcn_sched_barrier(0);
    };
    auto step = [&](auto full_tag, int j, SBlk& s_in, SBlk& s_out) __attribute__((always_inline)) {
      if constexpr (decltype(full_tag)::value)
        full_step(j, s_in, s_out);
      else
        part_step(j, s_in, s_out);
    };
    typedef std::integral_constant<bool, true> Full;
    typedef std::integral_constant<bool, false> Part;


    // Tile t covers steps 2t and 2t+1, which read tiles t and t+1. Tile t+3
    // is issued into the buffer of tile t-1 (free since the last barrier);
    // tile t+2 lands and is converted before the barrier that ends tile t,
    // while tile t+3 stays in flight.
    auto tile = [&](auto full_tag, int t) __attribute__((always_inline)) {
      const bool more = t + 3 < n_tiles;
      if (more) issue_tile(t + 3);
      step(full_tag, 2 * t, sa, sb);
      step(full_tag, 2 * t + 1, sb, sa);
      if (t + 2 < n_tiles && t > 0) {
        if (more)
          wait_tiles<kDmaPerTile>();
        else
          wait_tiles<0>();
        convert_tile(t + 2);
      }
      tile_barrier();
    };
    // Tile 0 (no PV yet), full tiles (both steps complete and unmasked), then
    // the tail.
    const int t_full_end = min(n_tiles - 1, (first_masked / 2 - part + kP - 1) / kP);
    tile(Part{}, 0);
    int t = 1;
    for (; t < t_full_end; ++t) tile(Full{}, t);
    for (; t < n_tiles; ++t) tile(Part{}, t);
    pv(va, pb);  // the last step's weights
  }
  if constexpr (KH == 2) {
    // The halves meet at equally many barriers: the one with fewer tiles
    // waits out the other's (the prologue's barrier, then one per tile).
    const int mine = n_tiles > 0 ? 1 + n_tiles : 0;
    const int most = t_most > 0 ? 1 + t_most : 0;
    for (int i = mine; i < most; ++i) tile_barrier();
    // No wave reads a tile any more and every tile load has landed. Half h
    // keeps, and will write, the 32 output columns of its accumulator block h
    // (d 32h..32h+31): it leaves the other block of its O in its own V ring
    // and its max and sum in its own K ring ([wave][block][register][lane]),
    // and after a barrier folds the other half's values for its block into
    // its own by the log-sum-exp rule (exp2 domain), taking the halves in
    // order, so both compute the same sums. A half without keys holds the
    // initial max and zero sums.
    constexpr int kRing = kNB * kTileH;  // 16-bit elements of one half's K or V ring
    static_assert(QW * kQB * 16 * 64 * 4 <= kRing * 2, "O block fits a ring");
    static_assert(QW * kQB * 2 * 64 * 4 <= kRing * 2, "max and sum fit a ring");
    float* const xo_mine = reinterpret_cast<float*>(Vs + half * kRing);
    float* const xm_mine = reinterpret_cast<float*>(Ks + half * kRing);
    const float* const xo_other = reinterpret_cast<const float*>(Vs + (1 - half) * kRing);
    const float* const xm_other = reinterpret_cast<const float*>(Ks + (1 - half) * kRing);
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      float* const po = xo_mine + (wq * kQB + j) * 16 * 64 + lane;
      if (half == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) po[i * 64] = o[j][1][i];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) po[i * 64] = o[j][0][i];
      }
      xm_mine[((wq * kQB + j) * 2) * 64 + lane] = m[j];
      xm_mine[((wq * kQB + j) * 2 + 1) * 64 + lane] = l[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      const float mx = xm_other[((wq * kQB + j) * 2) * 64 + lane];
      const float lx = xm_other[((wq * kQB + j) * 2 + 1) * 64 + lane];
      const float m0 = half == 0 ? m[j] : mx, m1 = half == 0 ? mx : m[j];
      const float l0 = half == 0 ? l[j] : lx, l1 = half == 0 ? lx : l[j];
      const float mm = fmaxf(m0, m1);
      const float e0 = __builtin_amdgcn_exp2f(m0 - mm), e1 = __builtin_amdgcn_exp2f(m1 - mm);
      l[j] = l0 * e0 + l1 * e1;
      const float* const px = xo_other + (wq * kQB + j) * 16 * 64 + lane;
      if (half == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[j][0][i] = o[j][0][i] * e0 + px[i * 64] * e1;
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[j][1][i] = px[i * 64] * e0 + o[j][1][i] * e1;
      }
      m[j] = mm;
    }
    // The output staging below reuses the rings.
    __syncthreads();
  }
  if constexpr (WS > 1) {
    // The block's workgroups each publish every wave's (O block, max, sum),
    // lane by lane, as agent-scope stores; after every wave has waited for
    // its stores, one thread counts the workgroup in. The workgroup that
    // counts last folds the partials (log-sum-exp, exp2 domain), re-arms the
    // counter and writes the output; the others are done. The fold takes the
    // partials in split order whichever workgroup runs it, so the bits do not
    // depend on which one finishes last.
    constexpr int kPart = kSplitPartWg;
    const int pw = (half * kWaves + wq) * kSplitPartWave + lane;
    {
      float* const p = a.split_part + (static_cast<int64_t>(blk) * WS + wsplit) * kPart + pw;
      auto publish = [&](const f32x16& ob) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) st_agent(p + i * 64, ob[i]);
      };
      if (half == 0)
        publish(o[0][0]);
      else
        publish(o[0][1]);
      st_agent(p + 16 * 64, m[0]);
      st_agent(p + 17 * 64, l[0]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned* const counter = a.split_counters + static_cast<int64_t>(blk) * kSplitCounterStride;
    if (tid == 0)
      merger = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               static_cast<unsigned>(WS - 1);
    __syncthreads();
    if (!merger) return;
    {
      // The other workgroups' partials; split s's is (m_s, l_s, O_s).
      float px[WS][16], pm[WS], pl[WS];
#pragma unroll
      for (int s2 = 0; s2 < WS; ++s2) {
        pm[s2] = pl[s2] = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) px[s2][i] = 0.f;
        if (s2 == wsplit) continue;
        const float* const p = a.split_part + (static_cast<int64_t>(blk) * WS + s2) * kPart + pw;
#pragma unroll
        for (int i = 0; i < 16; ++i) px[s2][i] = ld_agent(p + i * 64);
        pm[s2] = ld_agent(p + 16 * 64);
        pl[s2] = ld_agent(p + 17 * 64);
      }
      float ms[WS], e[WS];
#pragma unroll
      for (int s2 = 0; s2 < WS; ++s2) ms[s2] = s2 == wsplit ? m[0] : pm[s2];
      float mm = ms[0];
#pragma unroll
      for (int s2 = 1; s2 < WS; ++s2) mm = fmaxf(mm, ms[s2]);
#pragma unroll
      for (int s2 = 0; s2 < WS; ++s2) e[s2] = __builtin_amdgcn_exp2f(ms[s2] - mm);
      float lsum = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < WS; ++s2) lsum += (s2 == wsplit ? l[0] : pl[s2]) * e[s2];
      auto fold = [&](f32x16& ob) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float v = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < WS; ++s2) v += (s2 == wsplit ? ob[i] : px[s2][i]) * e[s2];
          ob[i] = v;
        }
      };
      if (half == 0)
        fold(o[0][0]);
      else
        fold(o[0][1]);
      l[0] = lsum;
      m[0] = mm;
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Sum of this lane's outputs: inf/NaN when any of them is.
  float chk = 0.f;
  // The wave's first query.
  const int qw = qblk * kM + wq * (32 * kQB);
  if constexpr (KH == 1) {
    // The outputs leave as whole 256-byte query rows. Each wave stages its
    // 32*QB rows in the LDS tiles (no longer read after the last tile
    // barrier, and every tile load has landed), 16-byte chunk c of row r at
    // c ^ (r % 16), then 16 lanes store one row: stored straight from the
    // MFMA layout, one instruction would write 32 bytes to each of 32 rows.
    constexpr int kStageBytes = 32 * kQB * 256;
    static_assert(QW * kStageBytes <= static_cast<int>(sizeof(Ks) + sizeof(Vs)), "staging fits");
    char* const stage = wq * kStageBytes < static_cast<int>(sizeof(Ks))
                            ? reinterpret_cast<char*>(Ks) + wq * kStageBytes
                            : reinterpret_cast<char*>(Vs) + (wq * kStageBytes - sizeof(Ks));
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      // l is the whole row sum in both lanes of the query (the row sums are).
      const float inv = (l[j] > 0.f) ? 1.f / l[j] : 0.f;
      const int rr = 32 * j + r32;  // row within the wave's block
      char* const srow = stage + rr * 256;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const f32x4 lo4 =
            f32x4{o[j][0][4 * gq], o[j][0][4 * gq + 1], o[j][0][4 * gq + 2], o[j][0][4 * gq + 3]} *
            inv;
        const f32x4 hi4 =
            f32x4{o[j][1][4 * gq], o[j][1][4 * gq + 1], o[j][1][4 * gq + 2], o[j][1][4 * gq + 3]} *
            inv;
        *reinterpret_cast<f32x4*>(srow + (((2 * gq + hl) ^ (rr & 15)) * 16)) = lo4;
        *reinterpret_cast<f32x4*>(srow + (((8 + 2 * gq + hl) ^ (rr & 15)) * 16)) = hi4;
        if constexpr (Elem<T>::kConvertV) {
          if (q0 + 32 * j < a.t_q)
            chk += (lo4[0] + lo4[1]) + (lo4[2] + lo4[3]) + (hi4[0] + hi4[1]) + (hi4[2] + hi4[3]);
        }
      }
    }
    // The wave reads back what its own lanes wrote: LDS operations of one
    // wave complete in order.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int c16 = lane & 15;
    float* const ob = a.o + b * a.lo.bs + h * a.lo.hs + 4 * c16;
#pragma unroll
    for (int k = 0; k < 8 * kQB; ++k) {
      const int rr = 4 * k + (lane >> 4);
      const f32x4 v = *reinterpret_cast<const f32x4*>(stage + rr * 256 + ((c16 ^ (rr & 15)) * 16));
      // Non-temporal: the output is not read again by this launch, and
      // streaming it past the caches keeps them for the K/V that the other
      // query blocks of each head still read.
      if (qw + rr < a.t_q)
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(ob + static_cast<int64_t>(qw + rr) * a.lo.rs));
    }
  } else {
    // Key halves: half h writes columns d 32h..32h+31 of its waves' rows as
    // 128-byte half rows, staged in its own K ring with 16-byte chunk c of
    // row r at c ^ ((r / 2) % 8) (a 16-lane phase of the writes covers 16
    // rows, two per 256-byte bank line, and of the reads two whole rows),
    // then 8 lanes store one half row.
    constexpr int kStageBytes = 32 * kQB * 128;
    static_assert(QW * kStageBytes <= kNB * kTileH * 2, "a half's rows fit its K ring");
    char* const stage = reinterpret_cast<char*>(Ks + half * (kNB * kTileH)) + wq * kStageBytes;
    auto put = [&](const f32x16& ov, int j) __attribute__((always_inline)) {
      const float inv = (l[j] > 0.f) ? 1.f / l[j] : 0.f;
      const int rr = 32 * j + r32;
      char* const srow = stage + rr * 128;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const f32x4 v4 =
            f32x4{ov[4 * gq], ov[4 * gq + 1], ov[4 * gq + 2], ov[4 * gq + 3]} * inv;
        *reinterpret_cast<f32x4*>(srow + (((2 * gq + hl) ^ ((rr >> 1) & 7)) * 16)) = v4;
        if constexpr (Elem<T>::kConvertV) {
          if (q0 + 32 * j < a.t_q) chk += (v4[0] + v4[1]) + (v4[2] + v4[3]);
        }
      }
    };
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      if (half == 0)
        put(o[j][0], j);
      else
        put(o[j][1], j);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int c8 = lane & 7;
    float* const ob = a.o + b * a.lo.bs + h * a.lo.hs + 32 * half + 4 * c8;
#pragma unroll
    for (int k = 0; k < 4 * kQB; ++k) {
      const int rr = 8 * k + (lane >> 3);
      const f32x4 v =
          *reinterpret_cast<const f32x4*>(stage + rr * 128 + ((c8 ^ ((rr >> 1) & 7)) * 16));
      if (qw + rr < a.t_q)
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(ob + static_cast<int64_t>(qw + rr) * a.lo.rs));
    }
  }
  if constexpr (Elem<T>::kConvertV) {
    // A bf16 V value of magnitude >= 65536 is inf after the f16 conversion and
    // turns the rows that meet it into inf/NaN (a finite sum that overflows
    // only costs a needless recompute). Then the whole workgroup recomputes its
    // queries from the bf16 inputs with the f32 block routine, in LDS
    // that the tiles no longer use. This file is built without NaN semantics,
    // under which isfinite, and a bit test the compiler recognizes as one,
    // become |x| == inf (false for NaN): the exponent bits are tested as an
    // integer that the compiler cannot trace to a float.
    uint32_t chk_bits = __builtin_bit_cast(uint32_t, chk);
    asm volatile("" : "+v"(chk_bits));
    const bool bad = (chk_bits & 0x7f800000u) == 0x7f800000u;
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) nonfinite = 1;
    __syncthreads();
    if (nonfinite) {
      auto& tl = *reinterpret_cast<f32blk::Tiles<2>*>(Ks);
      // Every wave runs the routine, 32 query rows each; where that covers
      // more rows than the workgroup holds (key halves), t_q clipped to the
      // workgroup's block leaves the extra waves empty (they only share the
      // routine's tile loads and barriers).
      constexpr int kNW = QW * KH;
      constexpr int kRows = 32 * kNW;
      PrefillArgs ab = a;
      if constexpr (kRows > kM) ab.t_q = min(a.t_q, qblk * kM + kM);
#pragma unroll
      for (int r0 = 0; r0 < kM; r0 += kRows)
        f32blk::fa2_block<__bf16, __bf16, 2, kNW>(ab, qblk * kM + r0, h, b, tl);
    }
  }
}

// K1s: key split for grids of 128-query workgroups that occupy fewer than
// half the CUs (one whisper-tiny or -base encoder window: 72 or 96 blocks).
// There, every wave of the 128-query kernel carries its 32 queries through
// all keys while most SIMDs idle. A key-split workgroup runs one 32-query block with 4 waves that
// take its 32-key steps in turn (step j on wave j % 4), each with its own
// online softmax, so a block's keys run on four SIMDs and the grid has four
// times the workgroups. The step arithmetic is K1's (S^T = K Q^T on 32x32x16
// MFMAs, weights exp2(c s - m) packed to f16, row sums on the matrix pipe,
// the same lazy rescale, O^T += V^T P^T); the operands move differently,
// since the waves share no keys: each wave loads its K rows straight into
// registers (a 16-byte load per lane and 16 d is the A-operand layout of the
// score MFMA) and moves its V rows into its own ring of four 32-key LDS slots
// with buffer_load ... lds (the transposed reads need them in LDS), three
// steps ahead of the step it computes. The waves then merge their (max, sum,
// O) in LDS by the log-sum-exp rule (exp2 domain).
constexpr int kKsQ = 32;                 // queries per key-split workgroup
constexpr int kKsRing = 4;               // V slots per wave; steps in flight
constexpr int kKsStepH = 32 * 64;        // 16-bit elements of one 32-key V step: 4 KiB
constexpr int kKsPitch = 68;             // merge rows: floats per query row of O

template <typename T>
__global__ __launch_bounds__(kThreads, 2) void fa2_prefill_d64_ks(PrefillArgs a, int n_qblk) {
  __shared__ __attribute__((aligned(128))) uint16_t Vr[kWaves * kKsRing * kKsStepH];
  __shared__ int nonfinite;  // bf16: some output of the workgroup is inf/NaN
  static_assert(sizeof(f32blk::Tiles<2>) <= sizeof(Vr), "f32 tiles fit in the V rings");
  static_assert(kKsQ * kKsPitch * 4 + 2 * kKsQ * 4 <= kKsRing * kKsStepH * 2,
                "a wave's merge rows fit in its ring");

  const int lid = __builtin_amdgcn_readfirstlane(xcd_remap(blockIdx.x, gridDim.x));
  const int qblk = lid % n_qblk;
  const int bh = lid / n_qblk;
  const int h = bh % a.n_heads;
  const int b = bh / a.n_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, hl = lane >> 5;
  if (tid == 0) nonfinite = 0;

  const T* qp = static_cast<const T*>(a.q) + b * a.lq.bs + h * a.lq.hs;
  const T* kp = static_cast<const T*>(a.k) + b * a.lk.bs + h * a.lk.hs;
  const T* vp = static_cast<const T*>(a.v) + b * a.lv.bs + h * a.lv.hs;

  // Every global load of this kernel is inline asm and waited for with
  // explicit vmcnt counts: K lands in registers while V lands in LDS by DMA,
  // and the compiler, counting only the loads it sees, would wait for later
  // steps' K too. A loaded register is read only after its wait and an empty
  // asm that redefines it.
  // This lane's query: column r32 of the block's S^T (the same in all waves).
  const int q0 = qblk * kKsQ + r32;
  u32x4 qf[4] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
  if (q0 < a.t_q) {
    const T* row = qp + static_cast<int64_t>(q0) * a.lq.rs + hl * 8;
#pragma unroll
    for (int dk = 0; dk < 4; ++dk)
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(qf[dk]) : "v"(row + dk * 16) : "memory");
  }
  int kv_end = a.t_kv;
  if (a.causal) {
    const int last = min(qblk * kKsQ + kKsQ, a.t_q) - 1 + a.q_pos_offset;
    kv_end = min(kv_end, last + 1);
  }
  const int nsteps = (kv_end + 31) / 32;
  // This wave's steps j = wave + 4 i, i < ni.
  const int ni = nsteps > wave ? (nsteps - wave + 3) / 4 : 0;
  // First 32-key step that needs a mask.
  int first_masked = a.t_kv / 32;
  if (a.causal) first_masked = min(first_masked, (qblk * kKsQ + a.q_pos_offset + 1) / 32);

  // K: lane (r32, hl) loads key 32 j + r32, d 16 dk + 8 hl .. +8, through a
  // range-checked buffer (keys past t_kv read as zero).
  const u32x4 krs = buffer_rsrc(kp, static_cast<uint32_t>(((a.t_kv - 1) * a.lk.rs + 64) * 2));
  const uint32_t kofs = static_cast<uint32_t>((r32 * a.lk.rs + 8 * hl) * 2);
  const uint32_t kstep = static_cast<uint32_t>(32 * a.lk.rs * 2);
  // V: 8 rows (1 KiB) per DMA, lane i carrying row i/8, chunk i%8 of them,
  // stored with K1's chunk swizzle.
  const u32x4 vrs = buffer_rsrc(vp, static_cast<uint32_t>(((a.t_kv - 1) * a.lv.rs + 64) * 2));
  uint32_t vofs[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int crow = 8 * r + (lane >> 3);
    vofs[r] = static_cast<uint32_t>((crow * a.lv.rs + (((lane & 7) ^ swz(crow)) * 8)) * 2);
  }
  const uint32_t vstep = static_cast<uint32_t>(32 * a.lv.rs * 2);
  const uint32_t ring = lds_addr(Vr) + wave * (kKsRing * kKsStepH * 2);
  u32x4 kr[kKsRing][4];  // K of the steps in flight, by ring slot
  auto issue = [&](int i) __attribute__((always_inline)) {
    const int j = wave + 4 * i;
    const int slot = i % kKsRing;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(ring + slot * (kKsStepH * 2));
#pragma unroll
    for (int r = 0; r < 4; ++r) dma16(vrs, dst + 1024 * r, vofs[r] + j * vstep);
    const uint32_t ko = kofs + j * kstep;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(kr[slot][0]) : "v"(ko), "s"(krs)
                 : "memory");
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:32" : "=v"(kr[slot][1])
                 : "v"(ko), "s"(krs) : "memory");
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:64" : "=v"(kr[slot][2])
                 : "v"(ko), "s"(krs) : "memory");
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:96" : "=v"(kr[slot][3])
                 : "v"(ko), "s"(krs) : "memory");
  };
  // After a wait that covers its loads: the registers of a slot hold K.
  auto landed = [&](int slot) __attribute__((always_inline)) {
    asm volatile("" : "+v"(kr[slot][0]), "+v"(kr[slot][1]), "+v"(kr[slot][2]), "+v"(kr[slot][3]));
  };
  // bf16 V -> f16 in place, once the step's rows have landed.
  auto convert = [&](int i) __attribute__((always_inline)) {
    if constexpr (Elem<T>::kConvertV) {
      uint16_t* base = Vr + (wave * kKsRing + i % kKsRing) * kKsStepH;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u32x4* p = reinterpret_cast<u32x4*>(base + r * 512 + lane * 8);
        *p = Elem<T>::to_f16(*p);
      }
    }
  };
  // V^T operands of step i (K1's transposed reads, on a 32-row slot).
  const int g4 = lane >> 4, t4 = lane & 15;
  const int vr0 = 4 * (g4 >> 1) + (t4 >> 2), vc0 = 2 * (g4 & 1) + ((t4 & 3) >> 1);
  const uint32_t voff0 = static_cast<uint32_t>(vr0 * 128 + ((vc0 ^ swz(vr0)) * 16) + 8 * (t4 & 1));
  auto vfetch = [&](int i, u32x2 (&va)[8]) __attribute__((always_inline)) {
    const uint32_t vb = ring + (i % kKsRing) * (kKsStepH * 2) + voff0;
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const uint32_t x = (vb ^ (64u * cc + 32u * e)) + 1024u * e;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) va[4 * k2 + 2 * cc + e] = read_tr_at(x + 2048u * k2);
      }
  };

  const float c = a.scale * kLog2e;
  f32x16 o[2] = {f32x16{}, f32x16{}};
  float m = kNoMax, l = 0.f;
  f32x16 sbuf[2];
  u32x4 pb[2];
  u32x2 va[8];
  f32x4 ls;
  auto qk = [&](const u32x4 (&ka)[4], f32x16& s) __attribute__((always_inline)) {
    s = f32x16{};
#pragma unroll
    for (int dk = 0; dk < 4; ++dk) s = Elem<T>::mfma(ka[dk], qf[dk], s);
  };
  auto mask = [&](int j, f32x16& s) __attribute__((always_inline)) {
    const int qpos = q0 + a.q_pos_offset;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kk = 32 * j + 8 * (i >> 2) + 4 * hl + (i & 3);
      s[i] = ((kk >= a.t_kv) | ((a.causal != 0) & (kk > qpos))) ? -INFINITY : s[i];
    }
  };
  auto weights = [&](const f32x16& s) __attribute__((always_inline)) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const f32x2 pp = {__builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * k2 + 2 * w], c, -m)),
                          __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * k2 + 2 * w + 1], c, -m))};
        pb[k2][w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pp, f16x2));
      }
  };
  const _Float16 rs_one = ((lane >> 2) & 1) == ((lane >> 4) & 1) ? 1.0f16 : 0.0f16;
  const f16x8 rs_sel = {rs_one, rs_one, rs_one, rs_one, rs_one, rs_one, rs_one, rs_one};
  auto row_sums = [&]() __attribute__((always_inline)) {
    const f32x4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
        rs_sel, __builtin_bit_cast(f16x8, pb[0]), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    ls = __builtin_amdgcn_mfma_f32_16x16x32_f16(rs_sel, __builtin_bit_cast(f16x8, pb[1]), acc, 0,
                                                0, 0);
  };
  auto pv = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const u32x4 v0 = {va[4 * k2].x, va[4 * k2].y, va[4 * k2 + 1].x, va[4 * k2 + 1].y};
      const u32x4 v1 = {va[4 * k2 + 2].x, va[4 * k2 + 2].y, va[4 * k2 + 3].x, va[4 * k2 + 3].y};
      o[0] = mfma_f16(v0, pb[k2], o[0]);
      o[1] = mfma_f16(v1, pb[k2], o[1]);
    }
  };
  // K1's lazy rescale on the step's intact scores (see the file header).
  auto settle = [&](const f32x16& s) __attribute__((always_inline)) {
    const bool need = __builtin_bit_cast(uint32_t, ls[0]) >
                      min(__builtin_bit_cast(uint32_t, l) + 0x00800000u,
                          __builtin_bit_cast(uint32_t, kSumLimit));
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      float mr = fmaxf(s[0], s[1]);
#pragma unroll
      for (int i = 2; i < 16; i += 2) mr = fmaxf(fmaxf(mr, s[i]), s[i + 1]);
      const float mx = pair_max(mr) * c;
      bool moved = false;
      if (mx > m) {
        const float alpha = __builtin_amdgcn_exp2f(m - mx);
        m = mx;
        l *= alpha;
        o[0] *= alpha;
        o[1] *= alpha;
        moved = true;
      }
      if (__builtin_amdgcn_ballot_w64(moved)) {
        weights(s);
        row_sums();
      }
    }
    l += ls[0];
  };
  auto wait_loads = [&](int i) __attribute__((always_inline)) {
    // K of step i+1 (and everything issued before it) has landed: the steps
    // issued after it, up to i+3, stay in flight.
    const int after = min(ni - 1, i + 3) - (i + 1);
    __builtin_amdgcn_sched_barrier(0);
    if (after >= 2)
      asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if (after == 1)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  if (ni > 0) {
    issue(0);
    if (ni > 1) issue(1);
    if (ni > 2) issue(2);
    // q and step 0 landed (steps 1 and 2 may still fly).
    wait_loads(-1);
    asm volatile("" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]));
    landed(0);
    convert(0);
    qk(kr[0], sbuf[0]);
    // Step i: P V of step i-1, step i+3's loads into the slot step i-1 used,
    // S of step i+1, the weights of step i, its V^T reads, its rescale check.
    auto step = [&](int i, f32x16& s_in, f32x16& s_out) __attribute__((always_inline)) {
      const int j = wave + 4 * i;
      if (i >= 1) pv();
      // The V^T reads of step i-1 have completed (P V waited for them), so
      // its slot may be overwritten.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (i + 3 < ni) issue(i + 3);
      if (i + 1 < ni) {
        wait_loads(i);
        landed((i + 1) % kKsRing);
        convert(i + 1);
        qk(kr[(i + 1) % kKsRing], s_out);
      }
      if (j >= first_masked) mask(j, s_in);
      if (i == 0) {
        // The reference max from the first two steps' (masked) scores, so
        // neither forms its weights twice.
        float mr = fmaxf(s_in[0], s_in[1]);
#pragma unroll
        for (int e = 2; e < 16; e += 2) mr = fmaxf(fmaxf(mr, s_in[e]), s_in[e + 1]);
        if (ni > 1) {
          if (j + 4 >= first_masked) mask(j + 4, s_out);
#pragma unroll
          for (int e = 0; e < 16; e += 2) mr = fmaxf(fmaxf(mr, s_out[e]), s_out[e + 1]);
        }
        const float mx = pair_max(mr) * c;
        if (mx > m) m = mx;
      }
      weights(s_in);
      row_sums();
      vfetch(i, va);
      __builtin_amdgcn_sched_barrier(0);
      settle(s_in);
      __builtin_amdgcn_sched_barrier(0);
    };
    // Unrolled by the ring length, so every ring index is a constant.
    for (int i0 = 0; i0 < ni; i0 += kKsRing) {
#pragma unroll
      for (int u = 0; u < kKsRing; ++u)
        if (i0 + u < ni) step(i0 + u, sbuf[u & 1], sbuf[(u + 1) & 1]);
    }
    pv();  // the last step's weights
  }

  // Merge: each wave leaves its O (query-major rows), max and sum in its own
  // ring, then thread t combines columns 4 (t % 16) .. +4 of queries t / 16
  // and t / 16 + 16, storing them as 16-byte pieces of whole output rows.
  // No load of this wave is in flight (a wave without keys has not waited for
  // its q loads yet), and every wave is done with its ring.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  float* const mw = reinterpret_cast<float*>(Vr + wave * kKsRing * kKsStepH);
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq)
      *reinterpret_cast<f32x4*>(mw + r32 * kKsPitch + 32 * hf + 8 * gq + 4 * hl) =
          f32x4{o[hf][4 * gq], o[hf][4 * gq + 1], o[hf][4 * gq + 2], o[hf][4 * gq + 3]};
  if (hl == 0) {
    mw[kKsQ * kKsPitch + r32] = m;
    mw[kKsQ * kKsPitch + kKsQ + r32] = l;
  }
  __syncthreads();
  float chk = 0.f;
  {
    const int c16 = tid & 15;
    float* const ob = a.o + b * a.lo.bs + h * a.lo.hs + 4 * c16;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int mq = (tid >> 4) + 16 * half;
      const int oq = qblk * kKsQ + mq;
      float M = kNoMax;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float* t = reinterpret_cast<const float*>(Vr + w * kKsRing * kKsStepH);
        M = fmaxf(M, t[kKsQ * kKsPitch + mq]);
      }
      float L = 0.f;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float* t = reinterpret_cast<const float*>(Vr + w * kKsRing * kKsStepH);
        // A wave without keys holds the initial max and zero sums.
        const float e = __builtin_amdgcn_exp2f(t[kKsQ * kKsPitch + mq] - M);
        L = __builtin_fmaf(e, t[kKsQ * kKsPitch + kKsQ + mq], L);
        acc += e * *reinterpret_cast<const f32x4*>(t + mq * kKsPitch + 4 * c16);
      }
      const f32x4 v = acc * ((L > 0.f) ? 1.f / L : 0.f);
      if (oq < a.t_q) {
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(ob + static_cast<int64_t>(oq) * a.lo.rs));
        if constexpr (Elem<T>::kConvertV) chk += (v[0] + v[1]) + (v[2] + v[3]);
      }
    }
  }
  if constexpr (Elem<T>::kConvertV) {
    // bf16 V of magnitude >= 65536 (inf after the f16 conversion): the
    // block's 32 queries are computed again with the f32 block routine, as
    // in K1 (the exponent bits tested as an integer, see K1).
    uint32_t chk_bits = __builtin_bit_cast(uint32_t, chk);
    asm volatile("" : "+v"(chk_bits));
    const bool bad = (chk_bits & 0x7f800000u) == 0x7f800000u;
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) nonfinite = 1;
    __syncthreads();
    if (nonfinite) {
      // The block routine's first 32-query wave takes this block: query rows
      // start at this block's first row, and at most 32 of them exist.
      PrefillArgs ab = a;
      ab.q = static_cast<const T*>(a.q) + static_cast<int64_t>(qblk) * kKsQ * a.lq.rs;
      ab.o = a.o + static_cast<int64_t>(qblk) * kKsQ * a.lo.rs;
      ab.t_q = min(kKsQ, a.t_q - qblk * kKsQ);
      ab.q_pos_offset = a.q_pos_offset + qblk * kKsQ;
      auto& tl = *reinterpret_cast<f32blk::Tiles<2>*>(Vr);
      f32blk::fa2_block<__bf16, __bf16, 2>(ab, 0, h, b, tl);
    }
  }
}

// Compute units of the current device, read once.
int64_t device_cus() {
  static const int64_t cus = [] {
    int dev = 0, n = 256;
    if (hipGetDevice(&dev) == hipSuccess)
      (void)hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    return static_cast<int64_t>(n);
  }();
  return cus;
}

template <int QB, int KH, int QW = kWaves, int WS = 1>
hipError_t launch_qb(const PrefillArgs& a, DType dt, hipStream_t s) {
  constexpr int kM = queries_per_wg<QB, QW>();
  const int n_qblk = (a.t_q + kM - 1) / kM;
  const int64_t nwg = n_qblk * static_cast<int64_t>(a.n_heads) * a.batch * WS;
  if (nwg > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nwg)), block(64 * QW * KH);
  if (dt == kF16)
    hipLaunchKernelGGL((fa2_prefill_d64<_Float16, QB, KH, QW, WS>), grid, block, 0, s, a, n_qblk);
  else
    hipLaunchKernelGGL((fa2_prefill_d64<__bf16, QB, KH, QW, WS>), grid, block, 0, s, a, n_qblk);
  return hipGetLastError();
}

}  // namespace

bool prefill_mfma16_supports(const PrefillArgs& a) {
  // K/V rows are addressed through 32-bit buffer offsets, and the range check
  // that zero-fills keys past t_kv needs rows at least one head wide.
  const int64_t span_k = (static_cast<int64_t>(a.t_kv) + kN) * a.lk.rs * 2;
  const int64_t span_v = (static_cast<int64_t>(a.t_kv) + kN) * a.lv.rs * 2;
  return a.d_head == 64 && a.lk.rs >= 64 && a.lv.rs >= 64 && span_k < (int64_t{1} << 31) &&
         span_v < (int64_t{1} << 31);
}

namespace {

// Workgroups per split block: as forced (-2 or -3), else three where that
// still fits one round of workgroups, else two.
int split_ways(const PrefillArgs& a, int64_t nwg1, int64_t cus) {
  if (a.force_queries == -2 || a.force_queries == -3) return -a.force_queries;
  return 3 * nwg1 <= cus ? 3 : 2;
}

// Scratch of a grid of nwg1 128-query blocks split `ways` ways.
int64_t split_floats(int64_t nwg1, int ways) { return nwg1 * ways * kSplitPartWg; }
int64_t split_words(int64_t nwg1) { return nwg1 * kSplitCounterStride; }

bool split_fits(const PrefillArgs& a, int64_t nwg1, int ways) {
  return a.split_part && a.split_counters &&
         split_floats(nwg1, ways) <= static_cast<int64_t>(a.split_part_floats) &&
         split_words(nwg1) <= static_cast<int64_t>(a.split_counter_words);
}

// Does the schedule split each 128-query block over several workgroups? By
// default for grids of fewer 128-query blocks than half the CUs (which then
// run two or three workgroups of 8 waves per block) over at least 1152 keys:
// one whisper-tiny window, 72 blocks, 12.5 against 18.2 us with the key split
// (three ways); one whisper-base window, 96 blocks, 14.4 against 18.2 us (two
// ways). Over fewer keys the merge through memory costs more than it saves
// (a whisper-tiny shape over 1024 frames: 10.9 against 9.2 us).
bool split_schedule(const PrefillArgs& a, int64_t nwg1, int64_t cus) {
  return a.force_queries == -2 || a.force_queries == -3 ||
         (a.force_queries == 0 && 2 * nwg1 < cus && a.t_kv >= 1152);
}

int64_t blocks128(const PrefillArgs& a) {
  constexpr int kM1 = queries_per_wg<1>();
  return ((a.t_q + kM1 - 1) / kM1) * static_cast<int64_t>(a.n_heads) * a.batch;
}

}  // namespace

void prefill_mfma16_scratch(const PrefillArgs& a, size_t* part_floats, size_t* counter_words) {
  const int64_t nwg1 = blocks128(a);
  const int64_t cus = device_cus();
  const bool used = a.t_q > 0 && nwg1 > 0 && split_schedule(a, nwg1, cus);
  *part_floats = used ? static_cast<size_t>(split_floats(nwg1, split_ways(a, nwg1, cus))) : 0;
  *counter_words = used ? static_cast<size_t>(split_words(nwg1)) : 0;
}

// The default schedule splits grids of at most one workgroup per CU.
size_t prefill_split_floats_min() { return static_cast<size_t>(device_cus()) * kSplitPartWg; }
size_t prefill_split_words_min() { return static_cast<size_t>(split_words(device_cus() / 2)); }

hipError_t launch_prefill_mfma16(const PrefillArgs& a, DType dt, hipStream_t s) {
  if (!prefill_mfma16_supports(a)) return hipErrorInvalidValue;
  const int64_t bh = static_cast<int64_t>(a.n_heads) * a.batch;
  if (bh <= 0 || a.t_q <= 0) return hipSuccess;
  // By the numbers n and n' of 128- and 192-query blocks (measured on encoder
  // windows, 1500 frames, one box):
  // - n > 2 per CU: 256-query workgroups, two per CU (large-v3 x4 windows,
  //   480 against 960 workgroups: 62.1 against 70.2 us);
  // - n > 1 per CU >= n': 192-query blocks on 12-wave workgroups whose halves
  //   split the keys, one per CU (whisper-base x4, 256 blocks: 27.7 against
  //   31.5 us with 128-query workgroups; whisper-small x2: 23.8 against 29.1).
  //   Three waves then share every SIMD, where 4-wave workgroups would leave
  //   CUs holding one of them alone;
  // - 1.25 per CU <= n <= 2 per CU otherwise: 256-query blocks on 8-wave
  //   key-halves workgroups (large-v3 x2: 35.1 against 36.4 us);
  // - 1 per CU < n < 1.25 per CU otherwise: 128-query workgroups, two per CU;
  // - half the CUs <= n <= 1 per CU: 128-query blocks on 8-wave workgroups
  //   with key halves (one large-v3 window, 240 blocks: 21.5 against 25.7 us;
  //   one whisper-small window, 144 blocks: 18.6 against 21.4);
  // - fewer, over at least 1152 keys: each block on two or three such
  //   workgroups, each over its share of the keys, merged through memory
  //   (split_schedule);
  // - fewer otherwise: the key split (32-query workgroups), which spreads a
  //   block over four CUs. It streams a block's K/V per 32 queries, 4x the
  //   bytes per FLOP of the 128-query kernel, which caps it near 50 GB/s per
  //   CU.
  // Below two blocks per CU a launch is one round of workgroups (~20-30 us),
  // in which each workgroup's fixed costs (q and the first tiles, the output
  // rows) are not hidden. a.force_queries forces one schedule: 256 or 128
  // queries per 4-wave workgroup, -256, -192 or -128 that many on 8 or 12
  // waves with key halves, -2 or -3 the split blocks over that many
  // workgroups, 32 the key split.
  constexpr int kM1 = queries_per_wg<1>();
  constexpr int kM6 = queries_per_wg<1, 6>();
  const int64_t nwg1 = ((a.t_q + kM1 - 1) / kM1) * bh;
  const int64_t nwg6 = ((a.t_q + kM6 - 1) / kM6) * bh;
  const int64_t cus = device_cus();
  const bool by_grid = a.force_queries == 0;
  if (a.force_queries == 256 || (by_grid && nwg1 > 2 * cus)) return launch_qb<2, 1>(a, dt, s);
  if (a.force_queries == -192 || (by_grid && nwg1 > cus && nwg6 <= cus))
    return launch_qb<1, 2, 6>(a, dt, s);
  if (a.force_queries == -256 || (by_grid && 4 * nwg1 >= 5 * cus))
    return launch_qb<2, 2>(a, dt, s);
  if (a.force_queries == 128 || (by_grid && nwg1 > cus)) return launch_qb<1, 1>(a, dt, s);
  if (a.force_queries == -128 || (by_grid && 2 * nwg1 >= cus)) return launch_qb<1, 2>(a, dt, s);
  if (split_schedule(a, nwg1, cus)) {
    const int ways = split_ways(a, nwg1, cus);
    if (split_fits(a, nwg1, ways))
      return ways == 3 ? launch_qb<1, 2, kWaves, 3>(a, dt, s) : launch_qb<1, 2, kWaves, 2>(a, dt, s);
    // No scratch (a call under stream capture before any outside it): the
    // key split below, unless forced.
    if (!by_grid) return hipErrorInvalidValue;
  }
  const int n_qblk = (a.t_q + kKsQ - 1) / kKsQ;
  const int64_t nwg = n_qblk * bh;
  if (nwg > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (dt == kF16)
    hipLaunchKernelGGL((fa2_prefill_d64_ks<_Float16>), dim3(static_cast<unsigned>(nwg)),
                       dim3(kThreads), 0, s, a, n_qblk);
  else
    hipLaunchKernelGGL((fa2_prefill_d64_ks<__bf16>), dim3(static_cast<unsigned>(nwg)),
                       dim3(kThreads), 0, s, a, n_qblk);
  return hipGetLastError();
}

}  // namespace wrs

