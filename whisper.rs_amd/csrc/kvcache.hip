// K3: device KV arena kernels (the storage side of
// crates/whisper/src/decoder.rs:131-264 DecoderKvCache).
//
// The arena keeps planes of [ctx][64] per (layer, slot, head) for
// self-attention and per (layer, head) for cross-attention, in f16 (default)
// or f32. These kernels convert or copy the decoder's f32 projection rows into
// that layout and move rows within / between planes; the row moves see an
// f32 row as two f16-sized rows.
#include "wrs_internal.hpp"

namespace wrs {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// One thread per 8 values: row i, head h, 8-column group c.
__global__ void kv_write_rows(const float* src, int64_t src_rs, int n, int n_heads,
                              _Float16* dst, int64_t dst_hs, int pos) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(n) * n_heads * 8;
  if (t >= total) return;
  const int c = static_cast<int>(t & 7);
  const int64_t ih = t >> 3;
  const int h = static_cast<int>(ih % n_heads);
  const int i = static_cast<int>(ih / n_heads);
  const float* s = src + static_cast<int64_t>(i) * src_rs + h * 64 + c * 8;
  f32x8 x;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = s[e];
  const f16x8 y = __builtin_convertvector(x, f16x8);
  *reinterpret_cast<f16x8*>(dst + h * dst_hs + static_cast<int64_t>(pos + i) * 64 + c * 8) = y;
}

// f32 planes: one thread per 4 values (row i, head h, 4-column group c). The
// source rows need only 4-byte alignment; the plane rows are 256-byte aligned.
__global__ void kv_write_rows_f32(const float* src, int64_t src_rs, int n, int n_heads,
                                  float* dst, int64_t dst_hs, int pos) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(n) * n_heads * 16;
  if (t >= total) return;
  const int c = static_cast<int>(t & 15);
  const int64_t ih = t >> 4;
  const int h = static_cast<int>(ih % n_heads);
  const int i = static_cast<int>(ih / n_heads);
  const float* s = src + static_cast<int64_t>(i) * src_rs + h * 64 + c * 4;
  const f32x4 x = {s[0], s[1], s[2], s[3]};
  *reinterpret_cast<f32x4*>(dst + h * dst_hs + static_cast<int64_t>(pos + i) * 64 + c * 4) = x;
}

// One workgroup per plane. Rows move down in blocks of 32 rows (256 threads x
// 8 halves); every block is read before any thread writes it, and later blocks
// only read rows above everything written so far, so the in-place move is safe
// for any drop >= 1.
__global__ __launch_bounds__(256) void kv_slide(_Float16* base, int64_t layer_stride,
                                                int64_t plane_stride, int len, int drop) {
  _Float16* p = base + blockIdx.y * layer_stride + blockIdx.x * plane_stride;
  const int keep = len - drop;
  const int tid = threadIdx.x;
  for (int r0 = 0; r0 < keep; r0 += 32) {
    const int r = r0 + (tid >> 3);
    const int c = (tid & 7) * 8;
    u32x4 v = {0, 0, 0, 0};
    if (r < keep) v = *reinterpret_cast<const u32x4*>(p + static_cast<int64_t>(r + drop) * 64 + c);
    __syncthreads();
    if (r < keep) *reinterpret_cast<u32x4*>(p + static_cast<int64_t>(r) * 64 + c) = v;
    __syncthreads();
  }
}

// Copy rows [0, len) of every (layer, head) plane from one slot to another.
__global__ __launch_bounds__(256) void kv_copy_planes(const _Float16* src, _Float16* dst,
                                                      int64_t layer_stride,
                                                      int64_t plane_stride, int len) {
  const int64_t off = blockIdx.y * layer_stride + blockIdx.x * plane_stride;
  const u32x4* s = reinterpret_cast<const u32x4*>(src + off);
  u32x4* d = reinterpret_cast<u32x4*>(dst + off);
  const int n = len * 8;  // 16-byte units
  for (int i = threadIdx.x; i < n; i += 256) d[i] = s[i];
}

// Zero fill of a strided [batch][head][row][cols] f32 region (replaces
// memset nodes, which must not be recorded into captured graphs): one thread
// per value.
__global__ __launch_bounds__(256) void fill_zero_rows(float* base, int64_t bs, int64_t hs,
                                                      int64_t rs, int n_heads, int n_rows,
                                                      int cols) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_batch = static_cast<int64_t>(n_heads) * n_rows * cols;
  const int b = static_cast<int>(blockIdx.y);
  if (t >= per_batch) return;
  const int c = static_cast<int>(t % cols);
  const int64_t hr = t / cols;
  const int r = static_cast<int>(hr % n_rows);
  const int h = static_cast<int>(hr / n_rows);
  base[b * bs + h * hs + r * rs + c] = 0.f;
}

__global__ __launch_bounds__(256) void fill_zero_u32(unsigned* p, int64_t n) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < n) p[t] = 0u;
}

}  // namespace

hipError_t launch_fill_zero_rows(float* base, int64_t bs, int64_t hs, int64_t rs, int batch,
                                 int n_heads, int n_rows, int cols, hipStream_t s) {
  if (batch <= 0 || n_heads <= 0 || n_rows <= 0 || cols <= 0) return hipSuccess;
  if (batch > 65535) return hipErrorInvalidConfiguration;
  const int64_t per_batch = static_cast<int64_t>(n_heads) * n_rows * cols;
  const int64_t blocks = (per_batch + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(fill_zero_rows, dim3(static_cast<unsigned>(blocks), batch), dim3(256), 0, s,
                     base, bs, hs, rs, n_heads, n_rows, cols);
  return hipGetLastError();
}

hipError_t launch_fill_zero_u32(unsigned* p, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(fill_zero_u32, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

hipError_t launch_kv_write_rows(const float* src, int64_t src_rs, int n, int n_heads,
                                _Float16* dst, int64_t dst_hs, int pos, hipStream_t s) {
  const int64_t total = static_cast<int64_t>(n) * n_heads * 8;
  if (total <= 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kv_write_rows, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, src,
                     src_rs, n, n_heads, dst, dst_hs, pos);
  return hipGetLastError();
}

hipError_t launch_kv_write_rows_f32(const float* src, int64_t src_rs, int n, int n_heads,
                                    float* dst, int64_t dst_hs, int pos, hipStream_t s) {
  const int64_t total = static_cast<int64_t>(n) * n_heads * 16;
  if (total <= 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kv_write_rows_f32, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, src,
                     src_rs, n, n_heads, dst, dst_hs, pos);
  return hipGetLastError();
}

hipError_t launch_kv_slide(_Float16* base, int64_t layer_stride, int64_t plane_stride,
                           int n_layers, int n_heads, int len, int drop, hipStream_t s) {
  if (n_layers <= 0 || n_heads <= 0 || drop <= 0 || len <= drop) return hipSuccess;
  hipLaunchKernelGGL(kv_slide, dim3(n_heads, n_layers), dim3(256), 0, s, base, layer_stride,
                     plane_stride, len, drop);
  return hipGetLastError();
}

hipError_t launch_kv_copy_planes(const _Float16* src, _Float16* dst, int64_t layer_stride,
                                 int64_t plane_stride, int n_layers, int n_heads, int len,
                                 hipStream_t s) {
  if (n_layers <= 0 || n_heads <= 0 || len <= 0) return hipSuccess;
  hipLaunchKernelGGL(kv_copy_planes, dim3(n_heads, n_layers), dim3(256), 0, s, src, dst,
                     layer_stride, plane_stride, len);
  return hipGetLastError();
}

}  // namespace wrs
