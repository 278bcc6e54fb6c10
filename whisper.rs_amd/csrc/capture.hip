// Alignment-head capture: softmax cross-attention weights of selected heads
// (replaces crates/whisper/src/decoder.rs:796-828 capture_cross_attention_heads,
//  called per text layer from decoder.rs:709-721 for DTW word timestamps).
//
// K5 (capture_cross_f16<pass>): one workgroup per (query block, key chunk,
//   pair), placed so that every query block of a key chunk runs on the XCD
//   that chunk belongs to, and the chunk's K rows are fetched into one L2
//   only. A call small enough for four XCDs (at most 128 workgroups, one per
//   CU) uses four, so that the query rows, which every XCD in use reads, are
//   fetched four times instead of eight. Two launches of the same kernel, or one when the attention
//   pass over the same q and keys left its row statistics (pass 2 below). A
//   workgroup of 4 waves owns 16 query rows of
//   one (slot, head) pair and one chunk of 128 keys of that head's f16 cross
//   plane (wave w: key tiles 2w and 2w+1 of 16 keys). Splitting the keys over
//   workgroups is what makes this fast: one CU streams only ~40 GB/s, so a
//   workgroup that walked a whole 1500-key plane (192 KB) and wrote its 96 KB
//   of weights would need ~7 us on its own.
//   Scores run on the matrix pipe as S^T = K Q^T with 16x16x32 f16 MFMAs: the
//   K tile is the A operand as stored; each f32 query is scaled by a power of
//   two (so the row's largest element lies in [2^14, 2^15)) and split into
//   three f16 parts hi + mid + lo that sum to it (11 + 11 + 11 bits cover the
//   24-bit significand; parts below 2^-24 of the scaled row are dropped), so
//   every product is exact and only the f32 accumulation rounds, as in
//   dot_f32 (simd.rs:4-119). Scores are then taken to the exp2 domain,
//   s * log2(e) (one rounding), so that every exponential is one v_exp_f32.
//   Pass 0 writes each chunk's row maximum m_c and sum l_c of exp2(s - m_c).
//   Pass 1 issues the loads of its rows' chunk statistics first, recomputes
//   its chunk's scores (bit-identical to pass 0), merges the statistics
//   (M = max m_c, L = sum l_c exp2(m_c - M)) and writes
//   exp2(s - M) * (1 / L): the max / exp / sum / reciprocal-multiply of
//   softmax.rs:1-23 with the sum gathered per chunk. Each lane stores the 4
//   consecutive weights of its query column as one 16-byte write.
//   Pass 2 is pass 1 with the row's (M, L) read from the statistics the
//   attention kernel wrote for the same rows (wrs_attn_prefill_cross_lse):
//   those come from its own f32 score sums, whose order differs from this
//   kernel's exact-product sums, so weights agree with the two-pass ones to
//   ~1e-6 relative rather than bit for bit.
//
// capture_cross_f32: the same weights over f32 cross planes, scalar.
#include "wrs_internal.hpp"

namespace wrs {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = kCaptureRows;        // 16 queries: the MFMA's N
constexpr int kTileKeys = 16;              // the MFMA's M
constexpr int kTilesPerWave = 2;
constexpr int kChunkKeys = kCaptureChunk;  // 128 keys per workgroup
constexpr int kMergeBatch = 16;            // chunk statistics in flight per lane

static_assert(kRows == 16, "one 16x16x32 MFMA column per query");
static_assert(kChunkKeys == kWaves * kTilesPerWave * kTileKeys, "chunk = the waves' tiles");

__device__ inline f32x4 mfma16(const u32x4& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b, c, 0, 0, 0);
}
__device__ inline float pow2(int e) { return __builtin_bit_cast(float, (e + 127) << 23); }
__device__ inline int clamp_exp(int e) { return e < -126 ? -126 : (e > 127 ? 127 : e); }

// Workgroup p of a launch runs on XCD p mod 8 (the dispatcher's round robin).
// Of n_xcd XCDs in use, XCD x takes chunks x, x + n_xcd, ...: the grid holds
// 8 * ceil(n_chunks / n_xcd) chunk slots per (pair, block), and workgroups on
// an XCD not in use, or of a slot past the last chunk, return at once. The
// placement decides only which L2 fetches what.
constexpr int kXcds = 8;

template <int kPass>
__global__ __launch_bounds__(kThreads) void capture_cross_f16(CaptureArgs a, int n_blocks,
                                                               int n_chunks, int n_xcd) {
  const int n_slots = (n_chunks + n_xcd - 1) / n_xcd;  // chunk slots per XCD
  const int xcd = blockIdx.x % kXcds, k = blockIdx.x / kXcds;
  const int block = k % n_blocks;
  const int chunk = xcd + n_xcd * ((k / n_blocks) % n_slots);
  const int pair = k / (n_blocks * n_slots);
  if (xcd >= n_xcd || chunk >= n_chunks) return;
  __shared__ float red[kWaves][kRows];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15;  // query column of this lane (B operand, C column)
  const int g = lane >> 4;  // k-group of the operands; keys 4g..4g+3 of a C tile
  const int head = a.head[pair];
  const int row = block * kRows + n;
  const bool row_ok = row < a.n_tokens;
  const int n_audio = a.n_audio;
  const int tile0 = chunk * (kChunkKeys / kTileKeys) + wave * kTilesPerWave;

  // Chunk statistics of block `block`: [row in block][chunk] (max, sum).
  f32x2* stats = reinterpret_cast<f32x2*>(a.part) +
                 (static_cast<int64_t>(pair) * n_blocks + block) * kRows * n_chunks;
  // Pass 1: the first kMergeBatch statistics of this lane's row, loaded before
  // anything else so their latency hides behind the score computation.
  f32x2 sv[kMergeBatch];
  f32x2 row_ml = {-INFINITY, 0.0f};
  if (kPass == 2 && row_ok)
    row_ml = reinterpret_cast<const f32x2*>(a.lse)[static_cast<int64_t>(head) * a.n_tokens + row];
  if (kPass == 1) {
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j)
      sv[j] = j < n_chunks ? stats[n * n_chunks + j] : f32x2{-INFINITY, 0.0f};
  }

  // K tile loads: lane (key 16t + n, group g) reads dims 16g..16g+15 (32 bytes);
  // MFMA step s of a tile covers dims 16g + 8s + j in k-group g for both
  // operands, so each dot product sums all 64 dims once. Keys past n_audio
  // read the last key (their scores are never used).
  const _Float16* kp = a.k + head * a.kv_hs + g * 16;
  u32x4 kx[kTilesPerWave][2];
#pragma unroll
  for (int u = 0; u < kTilesPerWave; ++u) {
    const int key = min((tile0 + u) * kTileKeys + n, n_audio - 1);
    const u32x4* src = reinterpret_cast<const u32x4*>(kp + static_cast<int64_t>(key) * 64);
    kx[u][0] = src[0];
    kx[u][1] = src[1];
  }

  // Query dims 16g..16g+15 of row `row`, scaled and split into three f16 parts.
  float qv[16];
  if (row_ok) {
    const f32x4* src = reinterpret_cast<const f32x4*>(a.q + row * a.q_rs + head * 64 + g * 16);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const f32x4 x = src[v];
#pragma unroll
      for (int d = 0; d < 4; ++d) qv[4 * v + d] = x[d];
    }
  } else {
#pragma unroll
    for (int d = 0; d < 16; ++d) qv[d] = 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int d = 0; d < 16; ++d) amax = fmaxf(amax, fabsf(qv[d]));
  amax = fmaxf(amax, __shfl_xor(amax, 16));
  amax = fmaxf(amax, __shfl_xor(amax, 32));
  // 2^sh brings the row maximum (biased exponent e) into [2^14, 2^15); zero
  // rows keep 1, inf/NaN rows propagate. Scores are scaled back by 2^-sh.
  const int e_max = static_cast<int>((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xFF);
  const int sh = e_max == 0 ? 0 : clamp_exp(141 - e_max);
  const float up = pow2(sh);
  const float down = pow2(clamp_exp(-sh)) * a.scale_log2;
  f16x8 qh[2], qm[2], ql[2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = qv[8 * s + j] * up;
      const _Float16 h = static_cast<_Float16>(x);
      const float r1 = x - static_cast<float>(h);
      const _Float16 m = static_cast<_Float16>(r1);
      const float r2 = r1 - static_cast<float>(m);
      qh[s][j] = h;
      qm[s][j] = m;
      ql[s][j] = static_cast<_Float16>(r2);
    }

  // acc[u][i]: score of key 16(tile0 + u) + 4g + i for query column n.
  f32x4 acc[kTilesPerWave];
#pragma unroll
  for (int u = 0; u < kTilesPerWave; ++u) {
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      c = mfma16(kx[u][s], qh[s], c);
      c = mfma16(kx[u][s], qm[s], c);
      c = mfma16(kx[u][s], ql[s], c);
    }
    acc[u] = c * down;
  }
  auto key_of = [&](int u, int i) { return (tile0 + u) * kTileKeys + 4 * g + i; };

  if (kPass == 0) {
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kTilesPerWave; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (key_of(u, i) < n_audio) mx = fmaxf(mx, acc[u][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (g == 0) red[wave][n] = mx;
    __syncthreads();
    mx = red[0][n];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, red[w][n]);
    __syncthreads();  // every wave has read the maxima before red is reused
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < kTilesPerWave; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (key_of(u, i) < n_audio) sum += __builtin_amdgcn_exp2f(acc[u][i] - mx);
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    if (g == 0) red[wave][n] = sum;
    __syncthreads();
    if (tid < kRows) {  // wave 0, lane n == tid: mx is this row's chunk maximum
      float l = red[0][tid];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) l += red[w][tid];
      stats[tid * n_chunks + chunk] = f32x2{mx, l};
    }
    return;
  }

  // Pass 1: merge the row's chunk statistics (batches beyond the first fold in
  // online), write the normalized weights. Pass 2: the row's statistics as given.
  if (!row_ok) return;
  float M = row_ml.x, L = row_ml.y;
  for (int c0 = 0; kPass == 1 && c0 < n_chunks; c0 += kMergeBatch) {
    if (c0 > 0) {
#pragma unroll
      for (int j = 0; j < kMergeBatch; ++j)
        sv[j] = c0 + j < n_chunks ? stats[n * n_chunks + c0 + j] : f32x2{-INFINITY, 0.0f};
    }
    float Mb = M;
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) Mb = fmaxf(Mb, sv[j].x);
    if (c0 > 0) L *= __builtin_amdgcn_exp2f(M - Mb);
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j)
      if (c0 + j < n_chunks) L += sv[j].y * __builtin_amdgcn_exp2f(sv[j].x - Mb);
    M = Mb;
  }
  const float inv = 1.0f / L;
  float* dst = a.out + (static_cast<int64_t>(a.row_offset + row) * a.n_selected + a.slot[pair]) *
                           static_cast<int64_t>(n_audio);
  const bool vec = (n_audio & 3) == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0;
#pragma unroll
  for (int u = 0; u < kTilesPerWave; ++u) {
    const int key0 = key_of(u, 0);
    if (key0 >= n_audio) break;
    f32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __builtin_amdgcn_exp2f(acc[u][i] - M) * inv;
    if (vec) {
      *reinterpret_cast<f32x4*>(dst + key0) = w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (key0 + i < n_audio) dst[key0 + i] = w[i];
    }
  }
}

// Capture over f32 cross planes (the f32 arena), decoder.rs:814-825 as
// written: one workgroup per (query row, pair); f32 scores dot * scale go into
// the output row, then the row's max, exp, sum and reciprocal multiply
// (softmax.rs:1-23) run over it in place. Each thread revisits only the keys
// it scored, so only the reductions synchronize. No scratch.
__device__ inline float block_reduce_f32(float x, float* sh, bool is_max) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float y = __shfl_xor(x, o);
    x = is_max ? fmaxf(x, y) : x + y;
  }
  __syncthreads();  // the previous reduction's readers are done with sh
  if (lane == 0) sh[wave] = x;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = is_max ? fmaxf(r, sh[w]) : r + sh[w];
  return r;
}

__global__ __launch_bounds__(kThreads) void capture_cross_f32(CaptureArgs a) {
  __shared__ float qsh[64];
  __shared__ float sh[kWaves];
  const int row = blockIdx.x, pair = blockIdx.y, tid = threadIdx.x;
  const int head = a.head[pair];
  const int n_audio = a.n_audio;
  if (tid < 64) qsh[tid] = a.q[static_cast<int64_t>(row) * a.q_rs + head * 64 + tid];
  __syncthreads();
  float* dst = a.out + (static_cast<int64_t>(a.row_offset + row) * a.n_selected + a.slot[pair]) *
                           static_cast<int64_t>(n_audio);
  const float* kp = a.k32 + head * a.kv_hs;
  float mx = -INFINITY;
  for (int j = tid; j < n_audio; j += kThreads) {
    const f32x4* kr = reinterpret_cast<const f32x4*>(kp + static_cast<int64_t>(j) * 64);
    float dot = 0.0f;
#pragma unroll
    for (int d4 = 0; d4 < 16; ++d4) {
      const f32x4 kv = kr[d4];
#pragma unroll
      for (int e = 0; e < 4; ++e) dot = __builtin_fmaf(qsh[4 * d4 + e], kv[e], dot);
    }
    const float sc = dot * a.scale;
    dst[j] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = block_reduce_f32(mx, sh, true);
  float sum = 0.0f;
  for (int j = tid; j < n_audio; j += kThreads) {
    const float p = expf(dst[j] - mx);
    dst[j] = p;
    sum += p;
  }
  const float inv = 1.0f / block_reduce_f32(sum, sh, false);
  for (int j = tid; j < n_audio; j += kThreads) dst[j] *= inv;
}

}  // namespace

size_t capture_part_floats(int n_pairs, int n_tokens, int n_audio) {
  const size_t blocks = static_cast<size_t>((n_tokens + kRows - 1) / kRows);
  const size_t chunks = static_cast<size_t>((n_audio + kChunkKeys - 1) / kChunkKeys);
  return 2 * static_cast<size_t>(n_pairs) * blocks * kRows * chunks;
}

hipError_t launch_capture_cross_f16(const CaptureArgs& a, hipStream_t s) {
  if (a.n_tokens <= 0 || a.n_pairs <= 0 || a.n_audio <= 0) return hipSuccess;
  const int n_chunks = (a.n_audio + kChunkKeys - 1) / kChunkKeys;
  const int n_blocks = (a.n_tokens + kRows - 1) / kRows;
  const int64_t work = static_cast<int64_t>(n_chunks) * n_blocks * a.n_pairs;
  const int n_xcd = work <= 128 ? 4 : kXcds;
  const int64_t items =
      static_cast<int64_t>(kXcds) * ((n_chunks + n_xcd - 1) / n_xcd) * n_blocks * a.n_pairs;
  if (items > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(items));
  if (a.lse) {
    hipLaunchKernelGGL(capture_cross_f16<2>, grid, dim3(kThreads), 0, s, a, n_blocks, n_chunks, n_xcd);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(capture_cross_f16<0>, grid, dim3(kThreads), 0, s, a, n_blocks, n_chunks, n_xcd);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(capture_cross_f16<1>, grid, dim3(kThreads), 0, s, a, n_blocks, n_chunks, n_xcd);
  return hipGetLastError();
}

hipError_t launch_capture_cross_f32(const CaptureArgs& a, hipStream_t s) {
  if (a.n_tokens <= 0 || a.n_pairs <= 0 || a.n_audio <= 0) return hipSuccess;
  if (a.n_pairs > kMaxCapturePairs) return hipErrorInvalidValue;
  hipLaunchKernelGGL(capture_cross_f32, dim3(a.n_tokens, a.n_pairs), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace wrs
