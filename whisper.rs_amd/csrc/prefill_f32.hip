// K4: flash-attention prefill with f32 operands on gfx950 f32 MFMA
// (v_mfma_f32_32x32x2_f32), for the 1e-5 accumulate-check runs and for the
// shapes the 16-bit kernel does not take (d_head != 64, f32 queries against
// the f16 decoder cache). One workgroup runs one 128-query block
// (prefill_f32_block.hpp holds the block routine and its semantics).
#include "prefill_f32_block.hpp"

namespace wrs {
namespace {

using f32blk::fa2_block;
using f32blk::kM;
using f32blk::kThreads;
using f32blk::Tiles;

__device__ inline int xcd_remap(int pid, int nwg) {
  const int xcd = pid & 7, k = pid >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  return xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
}

template <typename QT, typename KT, int DB>
__global__ __launch_bounds__(kThreads, 1) void fa2_prefill_f32(PrefillArgs a, int n_qblk) {
  __shared__ Tiles<DB> tl;
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = lid / n_qblk;
  fa2_block<QT, KT, DB>(a, lid % n_qblk, bh % a.n_heads, bh / a.n_heads, tl);
}

template <typename QT, typename KT>
hipError_t launch_typed(const PrefillArgs& a, hipStream_t s) {
  const int n_qblk = (a.t_q + kM - 1) / kM;
  const int64_t nwg = static_cast<int64_t>(n_qblk) * a.n_heads * a.batch;
  if (nwg <= 0) return hipSuccess;
  if (nwg > 0x7fffffff) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<unsigned>(nwg)), block(kThreads);
  const int db = (a.d_head + 31) / 32;
  switch (db) {
    case 1: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 1>), grid, block, 0, s, a, n_qblk); break;
    case 2: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 2>), grid, block, 0, s, a, n_qblk); break;
    case 3: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 3>), grid, block, 0, s, a, n_qblk); break;
    case 4: hipLaunchKernelGGL((fa2_prefill_f32<QT, KT, 4>), grid, block, 0, s, a, n_qblk); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_f32(const PrefillArgs& a, DType q_dt, DType kv_dt, hipStream_t s) {
  if (q_dt == kF32 && kv_dt == kF32) return launch_typed<float, float>(a, s);
  if (q_dt == kF32 && kv_dt == kF16) return launch_typed<float, _Float16>(a, s);
  if (q_dt == kF16 && kv_dt == kF16) return launch_typed<_Float16, _Float16>(a, s);
  if (q_dt == kBF16 && kv_dt == kBF16) return launch_typed<__bf16, __bf16>(a, s);
  if (q_dt == kF32 && kv_dt == kBF16) return launch_typed<float, __bf16>(a, s);
  return hipErrorInvalidValue;
}

}  // namespace wrs
