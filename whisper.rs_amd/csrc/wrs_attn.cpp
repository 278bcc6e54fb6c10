// C-ABI runtime of the MI355X attention path: contexts (device + stream +
// scratch), host-slice drop-ins, device-resident prefill/decode dispatch and
// the device KV arena. Declarations and reference citations: include/wrs_attn.h.
#include "../../include/wrs_attn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "wrs_internal.hpp"

using wrs::DType;

// Fixed scratch of the allocation-free cross decode
// (wrs_attn_decode_cross_noalloc): kNoallocSlots slots, each f32 split-K
// partials followed by merge counters. Each GPU the library runs on holds its
// own copy until the process ends. A context claims one slot of its GPU on its
// first allocation-free call and releases it when destroyed, so the calls of
// different contexts never share partials or counters.
constexpr int kNoallocSlots = 4;
constexpr size_t kNoallocPartBytes = size_t{512} << 10;     // 131072 f32 partials per slot
constexpr size_t kNoallocCounterBytes = size_t{16} << 10;   // 128 counter lines per slot
constexpr size_t kNoallocSlotBytes = kNoallocPartBytes + kNoallocCounterBytes;
static __device__ __align__(256) unsigned char scratch[kNoallocSlots * kNoallocSlotBytes];

struct wrs_attn_ctx {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  std::mutex mu;
  std::string err;
  // Device scratch, grown on demand and kept for the context's lifetime.
  void* stage = nullptr;  // host-slice staging of q/k/v/out and score rows
  size_t stage_bytes = 0;
  float* part = nullptr;  // decode split partials
  size_t part_bytes = 0;
  unsigned* counters = nullptr;  // decode merge counters (kept zero between launches)
  size_t counter_bytes = 0;
  float* cap_part = nullptr;  // alignment-head capture chunk statistics
  size_t cap_part_bytes = 0;
  void* lin_x = nullptr;  // projections: split f16 rows of f32 activations + row scales
  size_t lin_x_bytes = 0;
  float* ln_x = nullptr;  // fused projections above the weight-stream size: normalized rows
  size_t ln_x_bytes = 0;
  float* exact_scores = nullptr;  // f32 arena attention: full score rows
  size_t exact_scores_bytes = 0;
  // 16-bit prefill blocks whose keys split over two workgroups: partials and
  // merge counters (kept zero between launches). Allocated at their first use
  // for at least kSplitScratchBlocks blocks, so that every grid the default
  // schedule splits fits and graphs captured later keep valid pointers.
  float* split_part = nullptr;
  size_t split_part_bytes = 0;
  unsigned* split_counters = nullptr;
  size_t split_counter_bytes = 0;
  // Prefill schedule overrides (wrs_attn_set_schedule).
  int prefill_queries = 0;
  int f32_split = -1;
  // Slot of the allocation-free entry point's fixed scratch held by this
  // context (-1: none yet).
  int noalloc_slot = -1;
};

struct wrs_kv {
  wrs_attn_ctx* ctx = nullptr;
  int dtype = WRS_F16;  // element type of every plane: WRS_F16 or WRS_F32
  size_t n_layers = 0, n_slots = 0, n_heads = 0, max_ctx = 0, n_audio_max = 0;
  void* k_self = nullptr;  // [layer][slot][head][max_ctx][64]
  void* v_self = nullptr;
  void* k_cross = nullptr;  // [layer][head][n_audio_max][64]
  void* v_cross = nullptr;
  std::vector<size_t> len;        // per slot: rows stored (reference t_past)
  std::vector<size_t> cross_len;  // per layer: n_audio of the stored cross K/V

  bool f32() const { return dtype == WRS_F32; }
  size_t esize() const { return f32() ? 4 : 2; }
  size_t d_model() const { return n_heads * 64; }
  size_t plane() const { return max_ctx * 64; }
  size_t self_off(size_t layer, size_t slot) const {
    return ((layer * n_slots + slot) * n_heads) * plane();
  }
  size_t cross_off(size_t layer) const { return layer * n_heads * n_audio_max * 64; }
  // Element `off` of a plane set, typed. words() views any plane set as
  // 16-bit words (an f32 row of 64 is two f16-sized rows), so the row moves
  // of kv_slide / kv_copy_planes serve both element types.
  static uint16_t* u16(void* p, size_t off = 0) { return static_cast<uint16_t*>(p) + off; }
  static float* f32p(void* p, size_t off = 0) { return static_cast<float*>(p) + off; }
  _Float16* words(void* p, size_t off = 0) const {
    return static_cast<_Float16*>(p) + off * (esize() / 2);
  }
  size_t word_scale() const { return esize() / 2; }
};

namespace {

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

int fail(wrs_attn_ctx* c, int code, const char* what, hipError_t e = hipSuccess) {
  if (c) {
    c->err = what;
    if (e != hipSuccess) {
      c->err += ": ";
      c->err += hipGetErrorString(e);
    }
  }
  return code;
}

#define WRS_HIP(c, expr)                                        \
  do {                                                          \
    hipError_t e_ = (expr);                                     \
    if (e_ != hipSuccess) return fail((c), WRS_EHIP, #expr, e_); \
  } while (0)

// True while the context's stream records a graph: no allocation, free or
// host synchronization may happen then.
bool capturing(wrs_attn_ctx* c) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(c->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// Grows a scratch buffer to at least `bytes`. Refused while the stream is
// capturing (a captured graph would keep the old pointer, and hipMalloc /
// hipFree cannot be recorded): size scratch with wrs_attn_reserve first.
// `zero` clears the new buffer with a fill kernel (never a memset node).
int grow(wrs_attn_ctx* c, void** p, size_t* cap, size_t bytes, bool zero) {
  if (*cap >= bytes) return WRS_OK;
  if (capturing(c))
    return fail(c, WRS_ECAPTURE,
                "context scratch would grow during stream capture: call wrs_attn_reserve first");
  size_t want = std::max(bytes, *cap * 2);
  if (*p) {
    // The buffer may still be read by work queued on the stream.
    WRS_HIP(c, hipStreamSynchronize(c->stream));
    WRS_HIP(c, hipFree(*p));
    *p = nullptr;
    *cap = 0;
  }
  if (hipMalloc(p, want) != hipSuccess) {
    *p = nullptr;
    return fail(c, WRS_ENOMEM, "hipMalloc of context scratch failed");
  }
  *cap = want;
  if (zero)
    WRS_HIP(c, wrs::launch_fill_zero_u32(static_cast<unsigned*>(*p),
                                         static_cast<int64_t>(want / sizeof(unsigned)), c->stream));
  return WRS_OK;
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool fits_int(size_t x) { return x <= 0x7fffffffu; }

// Host-slice staging area: carve f32 regions out of the context buffer.
struct Stage {
  std::vector<size_t> offs;
  size_t total = 0;
  size_t add(size_t floats) {
    offs.push_back(total);
    total += align_up(floats * sizeof(float), 256);
    return offs.size() - 1;
  }
};

float* stage_ptr(wrs_attn_ctx* c, const Stage& s, size_t i) {
  return reinterpret_cast<float*>(static_cast<char*>(c->stage) + s.offs[i]);
}

int run_exact(wrs_attn_ctx* c, const float* q, size_t q_floats, const float* k, const float* v,
              size_t kv_floats, float* out, size_t out_floats, int n_rows, int n_heads,
              int d_head, int64_t d_model, int row_limit0) {
  // Device copy of the inputs, exact-semantics kernel, copy back.
  const size_t max_keys = static_cast<size_t>(row_limit0) + n_rows - 1;
  Stage st;
  const size_t iq = st.add(q_floats), ik = st.add(kv_floats), iv = st.add(kv_floats);
  const size_t io = st.add(out_floats);
  const size_t is = st.add(static_cast<size_t>(n_rows) * n_heads * std::max<size_t>(max_keys, 1));
  int rc = grow(c, &c->stage, &c->stage_bytes, st.total, false);
  if (rc) return rc;
  float *dq = stage_ptr(c, st, iq), *dk = stage_ptr(c, st, ik), *dv = stage_ptr(c, st, iv);
  float *dout = stage_ptr(c, st, io), *ds = stage_ptr(c, st, is);
  WRS_HIP(c, hipMemcpyAsync(dq, q, q_floats * 4, hipMemcpyHostToDevice, c->stream));
  if (kv_floats) {
    WRS_HIP(c, hipMemcpyAsync(dk, k, kv_floats * 4, hipMemcpyHostToDevice, c->stream));
    WRS_HIP(c, hipMemcpyAsync(dv, v, kv_floats * 4, hipMemcpyHostToDevice, c->stream));
  }
  wrs::ExactArgs a{};
  a.q = dq;
  a.k = dk;
  a.v = dv;
  a.o = dout;
  a.q_rs = d_model;
  a.o_rs = d_model;
  a.kv_rs = d_model;
  a.kv_hs = d_head;
  a.n_rows = n_rows;
  a.n_heads = n_heads;
  a.d_head = d_head;
  a.rows_per_group = n_rows;
  a.n_groups = 1;
  a.limit_step = 1;
  a.goff[0] = 0;
  a.glen[0] = row_limit0;
  a.scale = 1.0f / std::sqrt(static_cast<float>(d_head));
  a.scores = ds;
  a.scores_stride = static_cast<int64_t>(std::max<size_t>(max_keys, 1));
  WRS_HIP(c, wrs::launch_decode_exact_f32(a, c->stream));
  WRS_HIP(c, hipMemcpyAsync(out, dout, out_floats * 4, hipMemcpyDeviceToHost, c->stream));
  WRS_HIP(c, hipStreamSynchronize(c->stream));
  return WRS_OK;
}

// Scratch for a prefill schedule that splits blocks over workgroups (pf
// floats of partials, cw counter words; 0 when it needs none). Outside capture
// it is allocated here, at least the size every default split needs (so that
// graphs captured later keep valid pointers), or grown for a forced schedule
// on a larger grid; during capture the kernels take another schedule when
// what exists does not fit. Hands the buffers to `a`.
int split_scratch(wrs_attn_ctx* c, size_t pf, size_t cw, wrs::PrefillArgs& a) {
  if (pf && !capturing(c)) {
    int rc = grow(c, reinterpret_cast<void**>(&c->split_part), &c->split_part_bytes,
                  std::max(pf, wrs::prefill_split_floats_min()) * sizeof(float), false);
    if (rc) return rc;
    rc = grow(c, reinterpret_cast<void**>(&c->split_counters), &c->split_counter_bytes,
              std::max(cw, wrs::prefill_split_words_min()) * sizeof(unsigned), true);
    if (rc) return rc;
  }
  a.split_part = c->split_part;
  a.split_part_floats = c->split_part_bytes / sizeof(float);
  a.split_counters = c->split_counters;
  a.split_counter_words = c->split_counter_bytes / sizeof(unsigned);
  return WRS_OK;
}

int prefill_impl(wrs_attn_ctx* c, int q_dtype, const void* q, const wrs_layout& lq, int kv_dtype,
                 const void* k, const wrs_layout& lk, const void* v, const wrs_layout& lv,
                 float* out, const wrs_layout& lo, size_t batch, size_t n_heads, size_t t_q,
                 size_t t_kv, size_t d_head, int causal, size_t q_pos_offset) {
  if (batch == 0 || n_heads == 0 || t_q == 0) return WRS_OK;
  if (!q || !out || (t_kv && (!k || !v))) return fail(c, WRS_EINVAL, "null tensor pointer");
  if (d_head == 0 || d_head > 128) return fail(c, WRS_EUNSUPPORTED, "d_head must be 1..128");
  if (!fits_int(batch) || !fits_int(n_heads) || !fits_int(t_q) || !fits_int(t_kv) ||
      !fits_int(q_pos_offset) || !fits_int(t_q + q_pos_offset))
    return fail(c, WRS_EINVAL, "dimension exceeds 2^31");
  const bool same16 = q_dtype == kv_dtype && (q_dtype == WRS_F16 || q_dtype == WRS_BF16);
  const bool q32 = q_dtype == WRS_F32 &&
                   (kv_dtype == WRS_F32 || kv_dtype == WRS_F16 || kv_dtype == WRS_BF16);
  if (!same16 && !q32) return fail(c, WRS_EUNSUPPORTED, "unsupported q/kv dtype combination");

  wrs::PrefillArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = out;
  a.lq = {lq.batch_stride, lq.head_stride, lq.row_stride};
  a.lk = {lk.batch_stride, lk.head_stride, lk.row_stride};
  a.lv = {lv.batch_stride, lv.head_stride, lv.row_stride};
  a.lo = {lo.batch_stride, lo.head_stride, lo.row_stride};
  a.batch = static_cast<int>(batch);
  a.n_heads = static_cast<int>(n_heads);
  a.t_q = static_cast<int>(t_q);
  a.t_kv = static_cast<int>(t_kv);
  a.d_head = static_cast<int>(d_head);
  a.causal = causal ? 1 : 0;
  a.q_pos_offset = static_cast<int>(q_pos_offset);
  a.scale = 1.0f / std::sqrt(static_cast<float>(d_head));
  a.force_queries = c->prefill_queries;
  a.force_f32_split = c->f32_split;

  if (t_kv == 0) {
    // attention.rs:93-96: zero output. Rows of out may be strided.
    WRS_HIP(c, wrs::launch_fill_zero_rows(out, lo.batch_stride, lo.head_stride, lo.row_stride,
                                          static_cast<int>(batch), static_cast<int>(n_heads),
                                          static_cast<int>(t_q), static_cast<int>(d_head),
                                          c->stream));
    return WRS_OK;
  }

  auto aligned16 = [](const void* p, const wrs_layout& l, int mult) {
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && l.batch_stride % mult == 0 &&
           l.head_stride % mult == 0 && l.row_stride % mult == 0;
  };
  if (same16 && d_head == 64 && aligned16(q, lq, 8) && aligned16(k, lk, 8) &&
      aligned16(v, lv, 8) && aligned16(out, lo, 4) && wrs::prefill_mfma16_supports(a)) {
    size_t pf = 0, cw = 0;
    wrs::prefill_mfma16_scratch(a, &pf, &cw);
    const int rc = split_scratch(c, pf, cw, a);
    if (rc) return rc;
    WRS_HIP(c, wrs::launch_prefill_mfma16(a, q_dtype == WRS_F16 ? wrs::kF16 : wrs::kBF16,
                                          c->stream));
    return WRS_OK;
  }
  size_t pf = 0, cw = 0;
  wrs::prefill_f32_scratch(a, &pf, &cw);
  const int rc = split_scratch(c, pf, cw, a);
  if (rc) return rc;
  WRS_HIP(c, wrs::launch_prefill_f32(a, static_cast<DType>(q_dtype), static_cast<DType>(kv_dtype),
                                     c->stream));
  return WRS_OK;
}

// Device addresses of `scratch`, one per GPU: the array's host-side name is
// not a device address, so kernels and fills only ever see these.
constexpr int kMaxNoallocDevices = 64;
struct NoallocScratch {
  std::mutex mu;
  unsigned char* ptr[kMaxNoallocDevices] = {};
  bool held[kMaxNoallocDevices][kNoallocSlots] = {};  // slots claimed by live contexts
};
NoallocScratch& noalloc_scratch() {
  static NoallocScratch s;
  return s;
}

// Once per device, with that device current (the caller holds a DeviceGuard):
// resolve the array's address on this GPU and clear its merge counters.
int noalloc_setup(wrs_attn_ctx* c) {
  if (c->device >= kMaxNoallocDevices) return WRS_OK;  // the entry point refuses later
  NoallocScratch& ns = noalloc_scratch();
  std::lock_guard<std::mutex> lk(ns.mu);
  if (ns.ptr[c->device]) return WRS_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) return fail(c, WRS_EHIP, "hipGetSymbolAddress(scratch)", e);
  unsigned char* base = static_cast<unsigned char*>(p);
  for (int k = 0; k < kNoallocSlots; ++k)
    WRS_HIP(c, wrs::launch_fill_zero_u32(
                   reinterpret_cast<unsigned*>(base + k * kNoallocSlotBytes + kNoallocPartBytes),
                   static_cast<int64_t>(kNoallocCounterBytes / 4), c->stream));
  WRS_HIP(c, hipStreamSynchronize(c->stream));
  ns.ptr[c->device] = base;
  return WRS_OK;
}

// This context's slot of the fixed scratch, claimed on first use: nullptr
// with *rc set when the GPU has no fixed scratch or every slot is held.
unsigned char* noalloc_slot_ptr(wrs_attn_ctx* c, int* rc) {
  *rc = WRS_OK;
  if (c->device < 0 || c->device >= kMaxNoallocDevices) {
    *rc = fail(c, WRS_EUNSUPPORTED, "no fixed scratch on this device");
    return nullptr;
  }
  NoallocScratch& ns = noalloc_scratch();
  std::lock_guard<std::mutex> lk(ns.mu);
  if (!ns.ptr[c->device]) {
    *rc = fail(c, WRS_EUNSUPPORTED, "no fixed scratch on this device");
    return nullptr;
  }
  if (c->noalloc_slot < 0) {
    for (int k = 0; k < kNoallocSlots && c->noalloc_slot < 0; ++k)
      if (!ns.held[c->device][k]) {
        ns.held[c->device][k] = true;
        c->noalloc_slot = k;
      }
    if (c->noalloc_slot < 0) {
      *rc = fail(c, WRS_EBUSY,
                 "every slot of this GPU's fixed scratch is held by another context");
      return nullptr;
    }
  }
  return ns.ptr[c->device] + c->noalloc_slot * kNoallocSlotBytes;
}

void noalloc_release(wrs_attn_ctx* c) {
  if (c->noalloc_slot < 0 || c->device < 0 || c->device >= kMaxNoallocDevices) return;
  NoallocScratch& ns = noalloc_scratch();
  std::lock_guard<std::mutex> lk(ns.mu);
  ns.held[c->device][c->noalloc_slot] = false;
  c->noalloc_slot = -1;
}

// Split-K decode over f16 planes. `fixed` (the device address of `scratch`)
// replaces the context's scratch and is never grown: shapes whose partials or
// counters do not fit fail with WRS_ERANGE.
int decode_impl(wrs_attn_ctx* c, const float* q, int64_t q_rs, float* out, int64_t o_rs,
                const uint16_t* kbase, const uint16_t* vbase, int64_t kv_hs,
                const std::vector<int64_t>& goff, const std::vector<int>& lens, int rows_per_group,
                int n_heads, unsigned char* fixed = nullptr, float* lse = nullptr,
                int lse_rows = 0, int lse_row0 = 0) {
  const int n_groups = static_cast<int>(goff.size());
  if (n_groups == 0) return WRS_OK;
  if (!kbase || !vbase) return fail(c, WRS_EINVAL, "decode over an unallocated K/V plane");
  if (n_groups > wrs::kMaxDecodeGroups || rows_per_group < 1 ||
      rows_per_group > wrs::kMaxRowsPerGroup)
    return fail(c, WRS_EINVAL, "decode batch shape");
  wrs::DecodeArgs a{};
  a.q = q;
  a.o = out;
  a.k = reinterpret_cast<const _Float16*>(kbase);
  a.v = reinterpret_cast<const _Float16*>(vbase);
  a.q_rs = q_rs;
  a.o_rs = o_rs;
  a.kv_hs = kv_hs;
  int max_len = 0;
  for (int g = 0; g < n_groups; ++g) {
    a.goff[g] = goff[g];
    a.len[g] = lens[g];
    max_len = std::max(max_len, lens[g]);
  }
  a.n_groups = n_groups;
  a.rows_per_group = rows_per_group;
  a.n_heads = n_heads;
  // Sequences of 129..256 keys take one 256-key workgroup per (group, head):
  // no partials and no merge. Longer ones split into 128-key workgroups.
  a.chunk = (max_len > wrs::kDecodeChunk && max_len <= wrs::kDecodeChunkLong)
                ? wrs::kDecodeChunkLong
                : wrs::kDecodeChunk;
  a.n_splits = std::max(1, (max_len + a.chunk - 1) / a.chunk);
  a.scale_log2 = 0.125f * 1.4426950408889634f;
  a.lse = lse;
  a.lse_rows = lse_rows;
  a.lse_row0 = lse_row0;
  if (a.n_splits > 1) {
    const size_t pb =
        wrs::decode_part_floats(n_groups, n_heads, a.n_splits, rows_per_group) * sizeof(float);
    const size_t cb = wrs::decode_counter_words(n_groups, n_heads) * sizeof(unsigned);
    if (fixed) {
      if (pb > kNoallocPartBytes || cb > kNoallocCounterBytes)
        return fail(c, WRS_ERANGE,
                    "decode shape needs more than one slot of the fixed scratch (512 KiB of "
                    "partials, counters for 128 heads)");
    } else {
      int rc = grow(c, reinterpret_cast<void**>(&c->part), &c->part_bytes, pb, false);
      if (rc) return rc;
      rc = grow(c, reinterpret_cast<void**>(&c->counters), &c->counter_bytes, cb, true);
      if (rc) return rc;
    }
  }
  if (fixed) {
    a.part = reinterpret_cast<float*>(fixed);
    a.counters = reinterpret_cast<unsigned*>(fixed + kNoallocPartBytes);
  } else {
    a.part = c->part;
    a.counters = c->counters;
  }
  WRS_HIP(c, wrs::launch_decode_f16(a, c->stream));
  return WRS_OK;
}

const float* to_device_f32(wrs_attn_ctx* c, const float* src, size_t floats, int on_host,
                           size_t stage_offset_bytes, int* rc) {
  *rc = WRS_OK;
  if (!on_host) return src;
  float* dst =
      reinterpret_cast<float*>(static_cast<char*>(c->stage) + stage_offset_bytes);
  hipError_t e = hipMemcpyAsync(dst, src, floats * 4, hipMemcpyHostToDevice, c->stream);
  if (e != hipSuccess) *rc = fail(c, WRS_EHIP, "hipMemcpyAsync host->device", e);
  return dst;
}

}  // namespace

extern "C" {

const char* wrs_attn_status_string(int status) {
  switch (status) {
    case WRS_OK: return "ok";
    case WRS_EINVAL: return "invalid argument (reference would panic)";
    case WRS_ENOMEM: return "out of memory";
    case WRS_EHIP: return "HIP runtime error";
    case WRS_EUNSUPPORTED: return "unsupported on the GPU path";
    case WRS_ERANGE: return "index or length outside the arena";
    case WRS_ECAPTURE: return "scratch would grow during graph capture (reserve it first)";
    case WRS_EBUSY: return "every slot of the fixed scratch is held by another context";
    default: return "unknown status";
  }
}

int wrs_attn_create(int device, wrs_attn_ctx** out) {
  if (!out) return WRS_EINVAL;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return WRS_EINVAL;
  auto* c = new (std::nothrow) wrs_attn_ctx();
  if (!c) return WRS_ENOMEM;
  c->device = device;
  DeviceGuard g(device);
  if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return WRS_EHIP;
  }
  c->stream = c->own_stream;
  // The fixed scratch serves only the allocation-free entry point: if it
  // cannot be set up, the context still serves every other call and that
  // entry point returns WRS_EUNSUPPORTED.
  if (noalloc_setup(c) != WRS_OK) c->err.clear();
  *out = c;
  return WRS_OK;
}

void wrs_attn_destroy(wrs_attn_ctx* c) {
  if (!c) return;
  DeviceGuard g(c->device);
  (void)hipStreamSynchronize(c->stream);
  if (c->stage) (void)hipFree(c->stage);
  if (c->part) (void)hipFree(c->part);
  if (c->counters) (void)hipFree(c->counters);
  if (c->cap_part) (void)hipFree(c->cap_part);
  if (c->lin_x) (void)hipFree(c->lin_x);
  if (c->ln_x) (void)hipFree(c->ln_x);
  if (c->exact_scores) (void)hipFree(c->exact_scores);
  if (c->split_part) (void)hipFree(c->split_part);
  if (c->split_counters) (void)hipFree(c->split_counters);
  if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
  noalloc_release(c);  // the stream is drained: no call uses the slot any more
  delete c;
}

int wrs_attn_set_stream(wrs_attn_ctx* c, void* s) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  hipStream_t ns = static_cast<hipStream_t>(s);
  if (ns != c->stream) {
    // Work queued on the old stream may still use the context's scratch:
    // drain it, unless either stream is recording a graph (a host wait is not
    // allowed then, and the caller orders the streams).
    DeviceGuard g(c->device);
    hipStreamCaptureStatus so = hipStreamCaptureStatusNone, sn = hipStreamCaptureStatusNone;
    const bool cap_old = hipStreamIsCapturing(c->stream, &so) == hipSuccess &&
                         so != hipStreamCaptureStatusNone;
    const bool cap_new =
        hipStreamIsCapturing(ns, &sn) == hipSuccess && sn != hipStreamCaptureStatusNone;
    if (!cap_old && !cap_new) WRS_HIP(c, hipStreamSynchronize(c->stream));
  }
  c->stream = ns;
  return WRS_OK;
}

void* wrs_attn_get_stream(wrs_attn_ctx* c) { return c ? c->stream : nullptr; }

int wrs_attn_set_schedule(wrs_attn_ctx* c, int prefill_queries, int f32_split) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (prefill_queries != 0 && prefill_queries != 32 && prefill_queries != 128 &&
      prefill_queries != 256 && prefill_queries != -2 && prefill_queries != -3 &&
      prefill_queries != -128 &&
      prefill_queries != -192 && prefill_queries != -256)
    return fail(c, WRS_EINVAL,
                "prefill_queries must be 0, 32, 128, 256, -2, -3, -128, -192 or -256");
  if (f32_split < -1 || f32_split > 5)
    return fail(c, WRS_EINVAL, "f32_split must be -1..5");
  c->prefill_queries = prefill_queries;
  c->f32_split = f32_split;
  return WRS_OK;
}

int wrs_attn_synchronize(wrs_attn_ctx* c) {
  if (!c) return WRS_EINVAL;
  DeviceGuard g(c->device);
  WRS_HIP(c, hipStreamSynchronize(c->stream));
  return WRS_OK;
}

const char* wrs_attn_last_error(wrs_attn_ctx* c) { return c ? c->err.c_str() : "null context"; }

int wrs_stream_read(wrs_attn_ctx* c, const void* src, size_t bytes, float* sink,
                    size_t sink_len) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (bytes == 0) return WRS_OK;
  if (!src || !sink) return fail(c, WRS_EINVAL, "null argument");
  if (bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15))
    return fail(c, WRS_EINVAL, "stream_read: 16-byte aligned multiple of 16 bytes");
  if (sink_len < static_cast<size_t>(wrs::stream_read_blocks(static_cast<int64_t>(bytes))))
    return fail(c, WRS_EINVAL, "stream_read: sink shorter than one float per workgroup");
  DeviceGuard g(c->device);
  WRS_HIP(c, wrs::launch_stream_read(src, static_cast<int64_t>(bytes), sink, c->stream));
  return WRS_OK;
}

int wrs_stream_read_shape(wrs_attn_ctx* c, const void* src, size_t bytes, int threads,
                          int loads_per_lane, float* sink, size_t sink_len) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (bytes == 0) return WRS_OK;
  if (!src || !sink) return fail(c, WRS_EINVAL, "null argument");
  if (bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15))
    return fail(c, WRS_EINVAL, "stream_read_shape: 16-byte aligned multiple of 16 bytes");
  if ((threads != 256 && threads != 512 && threads != 1024) ||
      (loads_per_lane != 1 && loads_per_lane != 2 && loads_per_lane != 4 && loads_per_lane != 8 &&
       loads_per_lane != 16 && loads_per_lane != 24))
    return fail(c, WRS_EINVAL, "stream_read_shape: threads 256/512/1024, loads 1/2/4/8/16/24");
  if (sink_len < static_cast<size_t>(wrs::stream_read_shape_blocks(static_cast<int64_t>(bytes),
                                                                   threads, loads_per_lane)))
    return fail(c, WRS_EINVAL, "stream_read_shape: sink shorter than one float per workgroup");
  DeviceGuard g(c->device);
  WRS_HIP(c, wrs::launch_stream_read_shape(src, static_cast<int64_t>(bytes), threads,
                                           loads_per_lane, sink, c->stream));
  return WRS_OK;
}

int wrs_attn_reserve(wrs_attn_ctx* c, const wrs_reserve* r) {
  if (!c || !r) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard g(c->device);
  if (!fits_int(r->n_heads) || !fits_int(r->decode_rows) || !fits_int(r->decode_keys) ||
      !fits_int(r->capture_tokens) || !fits_int(r->capture_keys) ||
      !fits_int(r->linear_tokens) || !fits_int(r->linear_n_in))
    return fail(c, WRS_EINVAL, "wrs_attn_reserve: size exceeds 2^31");
  int rc = WRS_OK;
  const int heads = static_cast<int>(r->n_heads);
  if (heads && r->decode_rows && r->decode_keys > static_cast<size_t>(wrs::kDecodeChunkLong)) {
    // One decode launch: groups x rows_per_group query rows (a self step's
    // slots, up to kMaxDecodeGroups; an utterance's beams, up to
    // kMaxRowsPerGroup; cross-attention prompt rows, up to kMaxDecodeGroups
    // groups of kMaxRowsPerGroup), each row's partials per split of
    // kDecodeChunk keys.
    const int rows = static_cast<int>(std::min<size_t>(
        r->decode_rows, static_cast<size_t>(wrs::kMaxDecodeGroups) * wrs::kMaxRowsPerGroup));
    const int groups = std::min(rows, wrs::kMaxDecodeGroups);
    const int splits = static_cast<int>((r->decode_keys + wrs::kDecodeChunk - 1) / wrs::kDecodeChunk);
    rc = grow(c, reinterpret_cast<void**>(&c->part), &c->part_bytes,
              wrs::decode_part_floats(rows, heads, splits, 1) * sizeof(float), false);
    if (rc) return rc;
    rc = grow(c, reinterpret_cast<void**>(&c->counters), &c->counter_bytes,
              wrs::decode_counter_words(groups, heads) * sizeof(unsigned), true);
    if (rc) return rc;
  }
  if (r->capture_tokens && r->capture_keys) {
    rc = grow(c, reinterpret_cast<void**>(&c->cap_part), &c->cap_part_bytes,
              wrs::capture_part_floats(wrs::kMaxCapturePairs, static_cast<int>(r->capture_tokens),
                                       static_cast<int>(r->capture_keys)) * sizeof(float),
              false);
    if (rc) return rc;
  }
  if (r->linear_tokens > static_cast<size_t>(wrs::kGemvMaxRows) && r->linear_n_in) {
    const size_t split_bytes =
        align_up(r->linear_tokens * wrs::kSplitParts * r->linear_n_in * 2, 256);
    rc = grow(c, &c->lin_x, &c->lin_x_bytes, split_bytes + r->linear_tokens * 4, false);
    if (rc) return rc;
    rc = grow(c, reinterpret_cast<void**>(&c->ln_x), &c->ln_x_bytes,
              r->linear_tokens * r->linear_n_in * sizeof(float), false);
    if (rc) return rc;
  }
  WRS_HIP(c, hipStreamSynchronize(c->stream));
  return WRS_OK;
}

int wrs_single_token_mha_d64(wrs_attn_ctx* c, const float* q, size_t q_len, const float* k,
                             size_t k_len, const float* v, size_t v_len, size_t t_kv,
                             size_t n_heads, size_t d_model, float* output, size_t output_len) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard g(c->device);
  // attention.rs:322-327 reads head h at h*64 of q/out and of every key row.
  const size_t span = n_heads * 64;
  if (span > d_model || q_len < span || output_len < span)
    return fail(c, WRS_EINVAL, "single_token_mha_d64: head span exceeds q/output/d_model");
  const size_t kv_need = t_kv ? (t_kv - 1) * d_model + span : 0;
  if (k_len < kv_need || v_len < kv_need)
    return fail(c, WRS_EINVAL, "single_token_mha_d64: k/v shorter than t_kv rows");
  if (!fits_int(t_kv) || !fits_int(n_heads)) return fail(c, WRS_EINVAL, "dimension exceeds 2^31");
  if (n_heads == 0) return WRS_OK;
  if (t_kv == 0) {
    std::memset(output, 0, span * sizeof(float));
    return WRS_OK;
  }
  return run_exact(c, q, span, k, v, kv_need, output, span, 1, static_cast<int>(n_heads), 64,
                   static_cast<int64_t>(d_model), static_cast<int>(t_kv));
}

int wrs_flash_attention_2(wrs_attn_ctx* c, const float* q, size_t q_len, const float* k,
                          size_t k_len, const float* v, size_t v_len, size_t t_q, size_t t_kv,
                          size_t n_heads, size_t d_model, int causal, float* output,
                          size_t output_len) {
  if (!c) return WRS_EINVAL;
  // attention.rs:79-88
  if (n_heads == 0) return fail(c, WRS_EINVAL, "n_heads must be non-zero");
  if (d_model % n_heads != 0) return fail(c, WRS_EINVAL, "d_model is not divisible by n_heads");
  if (q_len != t_q * d_model || k_len != t_kv * d_model || v_len != t_kv * d_model ||
      output_len != t_q * d_model)
    return fail(c, WRS_EINVAL, "flash_attention_2: slice length mismatch");
  const size_t d_head = d_model / n_heads;
  if (t_q == 0) return WRS_OK;  // :90-92
  if (t_kv == 0) {              // :93-96
    std::memset(output, 0, output_len * sizeof(float));
    return WRS_OK;
  }
  if (t_q == 1 && d_head == 64 && !causal)  // :102-105
    return wrs_single_token_mha_d64(c, q, q_len, k, k_len, v, v_len, t_kv, n_heads, d_model,
                                    output, output_len);
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard g(c->device);
  if (d_head > 128) return fail(c, WRS_EUNSUPPORTED, "d_head > 128");
  if (!fits_int(t_q) || !fits_int(t_kv) || !fits_int(n_heads))
    return fail(c, WRS_EINVAL, "dimension exceeds 2^31");
  Stage st;
  const size_t iq = st.add(q_len), ik = st.add(k_len), iv = st.add(v_len), io = st.add(output_len);
  int rc = grow(c, &c->stage, &c->stage_bytes, st.total, false);
  if (rc) return rc;
  float *dq = stage_ptr(c, st, iq), *dk = stage_ptr(c, st, ik), *dv = stage_ptr(c, st, iv);
  float* dout = stage_ptr(c, st, io);
  WRS_HIP(c, hipMemcpyAsync(dq, q, q_len * 4, hipMemcpyHostToDevice, c->stream));
  WRS_HIP(c, hipMemcpyAsync(dk, k, k_len * 4, hipMemcpyHostToDevice, c->stream));
  WRS_HIP(c, hipMemcpyAsync(dv, v, v_len * 4, hipMemcpyHostToDevice, c->stream));
  const int64_t dm = static_cast<int64_t>(d_model), dh = static_cast<int64_t>(d_head);
  const wrs_layout tq{0, dh, dm};
  rc = prefill_impl(c, WRS_F32, dq, tq, WRS_F32, dk, tq, dv, tq, dout, tq, 1, n_heads, t_q, t_kv,
                    d_head, causal, 0);
  if (rc) return rc;
  WRS_HIP(c, hipMemcpyAsync(output, dout, output_len * 4, hipMemcpyDeviceToHost, c->stream));
  WRS_HIP(c, hipStreamSynchronize(c->stream));
  return WRS_OK;
}

int wrs_multi_head_attention(wrs_attn_ctx* c, const float* q, size_t q_len, const float* k,
                             size_t k_len, const float* v, size_t v_len, size_t t_q, size_t t_kv,
                             size_t n_heads, size_t d_model, int causal, float* output,
                             size_t output_len) {
  // attention.rs:29-41 forwards unchanged.
  return wrs_flash_attention_2(c, q, q_len, k, k_len, v, v_len, t_q, t_kv, n_heads, d_model,
                               causal, output, output_len);
}

int wrs_mha_with_cache(wrs_attn_ctx* c, const float* q, size_t q_len, const float* k,
                       size_t k_len, const float* v, size_t v_len, size_t n_tokens,
                       size_t total_tokens, size_t t_past, size_t n_heads, size_t d_model,
                       float* output, size_t output_len) {
  if (!c) return WRS_EINVAL;
  if (n_heads == 0 || d_model % n_heads != 0)
    return fail(c, WRS_EINVAL, "mha_with_cache: n_heads must divide d_model");
  // decoder.rs:846-850
  if (q_len != n_tokens * d_model || k_len != total_tokens * d_model ||
      v_len != total_tokens * d_model || output_len != n_tokens * d_model)
    return fail(c, WRS_EINVAL, "mha_with_cache: slice length mismatch");
  const size_t d_head = d_model / n_heads;
  if (n_tokens == 0) return WRS_OK;
  // Query i reads scores[0..=t_past+i] of a total_tokens buffer (decoder.rs:862-866).
  if (t_past + n_tokens > total_tokens)
    return fail(c, WRS_EINVAL, "mha_with_cache: t_past + n_tokens exceeds total_tokens");
  if (n_tokens == 1 && d_head == 64)  // decoder.rs:852-855
    return wrs_single_token_mha_d64(c, q, q_len, k, k_len, v, v_len, t_past + 1, n_heads,
                                    d_model, output, output_len);
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard g(c->device);
  if (d_head > 128) return fail(c, WRS_EUNSUPPORTED, "d_head > 128");
  if (!fits_int(total_tokens) || !fits_int(n_tokens) || !fits_int(n_heads))
    return fail(c, WRS_EINVAL, "dimension exceeds 2^31");
  return run_exact(c, q, q_len, k, v, (t_past + n_tokens) * d_model, output, output_len,
                   static_cast<int>(n_tokens), static_cast<int>(n_heads),
                   static_cast<int>(d_head), static_cast<int64_t>(d_model),
                   static_cast<int>(t_past + 1));
}

int wrs_attn_prefill(wrs_attn_ctx* c, int q_dtype, const void* q, const wrs_layout* q_layout,
                     int kv_dtype, const void* k, const wrs_layout* k_layout, const void* v,
                     const wrs_layout* v_layout, float* out, const wrs_layout* out_layout,
                     size_t batch, size_t n_heads, size_t t_q, size_t t_kv, size_t d_head,
                     int causal, size_t q_pos_offset) {
  if (!c) return WRS_EINVAL;
  if (!q_layout || !k_layout || !v_layout || !out_layout)
    return fail(c, WRS_EINVAL, "null layout");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard g(c->device);
  return prefill_impl(c, q_dtype, q, *q_layout, kv_dtype, k, *k_layout, v, *v_layout, out,
                      *out_layout, batch, n_heads, t_q, t_kv, d_head, causal, q_pos_offset);
}

// ---------------------------------------------------------------- KV arena

}  // extern "C"

namespace {

// Rows [pos, pos + n) of every head plane of one plane set (element `off`
// on), from n f32 rows of d_model: converted to f16, or copied for f32 arenas.
int write_rows(wrs_attn_ctx* c, wrs_kv* kv, const float* src, int64_t src_rs, size_t n,
               void* base, size_t off, int64_t plane, size_t pos) {
  const int nh = static_cast<int>(kv->n_heads);
  if (kv->f32())
    WRS_HIP(c, wrs::launch_kv_write_rows_f32(src, src_rs, static_cast<int>(n), nh,
                                             wrs_kv::f32p(base, off), plane,
                                             static_cast<int>(pos), c->stream));
  else
    WRS_HIP(c, wrs::launch_kv_write_rows(src, src_rs, static_cast<int>(n), nh,
                                         static_cast<_Float16*>(base) + off, plane,
                                         static_cast<int>(pos), c->stream));
  return WRS_OK;
}

// Attention over f32 arena planes on the exact decode kernel (the reference's
// own single-token and cached-prompt arithmetic): n_rows query rows of d_model
// in groups of rows_per_group that share the plane set at element goff[g];
// row i of group g sees glen[g] + i * limit_step keys. At most
// kMaxExactGroups groups and 65535 rows per call.
int exact_arena(wrs_attn_ctx* c, wrs_kv* kv, const float* q, float* out, void* kbase,
                void* vbase, int64_t kv_hs, const std::vector<int64_t>& goff,
                const std::vector<int>& glen, int rows_per_group, int limit_step, int n_rows) {
  if (n_rows <= 0) return WRS_OK;
  const size_t groups = goff.size();
  int max_len = 1;
  for (size_t g = 0; g < groups; ++g)
    max_len = std::max(max_len, glen[g] + (rows_per_group - 1) * limit_step);
  const size_t bytes =
      static_cast<size_t>(n_rows) * kv->n_heads * static_cast<size_t>(max_len) * sizeof(float);
  int rc = grow(c, reinterpret_cast<void**>(&c->exact_scores), &c->exact_scores_bytes, bytes,
                false);
  if (rc) return rc;
  wrs::ExactArgs a{};
  a.q = q;
  a.k = static_cast<const float*>(kbase);
  a.v = static_cast<const float*>(vbase);
  a.o = out;
  a.q_rs = static_cast<int64_t>(kv->d_model());
  a.o_rs = a.q_rs;
  a.kv_rs = 64;
  a.kv_hs = kv_hs;
  a.n_rows = n_rows;
  a.n_heads = static_cast<int>(kv->n_heads);
  a.d_head = 64;
  a.rows_per_group = rows_per_group;
  a.n_groups = static_cast<int>(groups);
  a.limit_step = limit_step;
  a.scale = 0.125f;  // 1/sqrt(64) (attention.rs:255, decoder.rs:857)
  a.scores = c->exact_scores;
  a.scores_stride = max_len;
  for (size_t g = 0; g < groups; ++g) {
    a.goff[g] = goff[g];
    a.glen[g] = glen[g];
  }
  WRS_HIP(c, wrs::launch_decode_exact_f32(a, c->stream));
  return WRS_OK;
}

}  // namespace

extern "C" {

int wrs_kv_create_dtype(wrs_attn_ctx* c, size_t n_layers, size_t n_slots, size_t n_heads,
                        size_t max_ctx, size_t n_audio_max, int dtype, wrs_kv** out) {
  if (!c || !out) return WRS_EINVAL;
  *out = nullptr;
  if (n_layers == 0 || n_heads == 0 || max_ctx == 0 || !fits_int(max_ctx) ||
      !fits_int(n_audio_max) || !fits_int(n_slots))
    return fail(c, WRS_EINVAL, "wrs_kv_create: bad geometry");
  if (dtype != WRS_F16 && dtype != WRS_F32)
    return fail(c, WRS_EINVAL, "wrs_kv_create: arena dtype must be WRS_F16 or WRS_F32");
  if (dtype == WRS_F32 && !fits_int(2 * max_ctx))  // row moves count f16-sized rows
    return fail(c, WRS_EINVAL, "wrs_kv_create: bad geometry");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard g(c->device);
  auto* kv = new (std::nothrow) wrs_kv();
  if (!kv) return WRS_ENOMEM;
  kv->ctx = c;
  kv->dtype = dtype;
  kv->n_layers = n_layers;
  kv->n_slots = n_slots;
  kv->n_heads = n_heads;
  kv->max_ctx = max_ctx;
  kv->n_audio_max = n_audio_max;
  kv->len.assign(n_slots, 0);
  kv->cross_len.assign(n_layers, 0);
  const size_t self_bytes = n_layers * n_slots * n_heads * max_ctx * 64 * kv->esize();
  const size_t cross_bytes = n_layers * n_heads * n_audio_max * 64 * kv->esize();
  bool ok = true;
  if (self_bytes) {
    ok = ok && hipMalloc(&kv->k_self, self_bytes) == hipSuccess;
    ok = ok && hipMalloc(&kv->v_self, self_bytes) == hipSuccess;
  }
  if (cross_bytes) {
    ok = ok && hipMalloc(&kv->k_cross, cross_bytes) == hipSuccess;
    ok = ok && hipMalloc(&kv->v_cross, cross_bytes) == hipSuccess;
  }
  if (!ok) {
    for (void* p : {(void*)kv->k_self, (void*)kv->v_self, (void*)kv->k_cross, (void*)kv->v_cross})
      if (p) (void)hipFree(p);
    delete kv;
    return fail(c, WRS_ENOMEM, "wrs_kv_create: hipMalloc failed");
  }
  *out = kv;
  return WRS_OK;
}

int wrs_kv_create(wrs_attn_ctx* c, size_t n_layers, size_t n_slots, size_t n_heads,
                  size_t max_ctx, size_t n_audio_max, wrs_kv** out) {
  return wrs_kv_create_dtype(c, n_layers, n_slots, n_heads, max_ctx, n_audio_max, WRS_F16, out);
}

int wrs_kv_dtype(wrs_kv* kv, int* dtype) {
  if (!kv || !dtype) return WRS_EINVAL;
  *dtype = kv->dtype;
  return WRS_OK;
}

void wrs_kv_destroy(wrs_kv* kv) {
  if (!kv) return;
  wrs_attn_ctx* c = kv->ctx;
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard g(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (void* p : {(void*)kv->k_self, (void*)kv->v_self, (void*)kv->k_cross, (void*)kv->v_cross})
    if (p) (void)hipFree(p);
  delete kv;
}

int wrs_kv_clear(wrs_kv* kv) {
  if (!kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  std::fill(kv->len.begin(), kv->len.end(), 0);
  return WRS_OK;
}

int wrs_kv_clear_slot(wrs_kv* kv, size_t slot) {
  if (!kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  if (slot >= kv->n_slots) return fail(kv->ctx, WRS_ERANGE, "slot out of range");
  kv->len[slot] = 0;
  return WRS_OK;
}

int wrs_kv_invalidate_cross(wrs_kv* kv) {
  if (!kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  std::fill(kv->cross_len.begin(), kv->cross_len.end(), 0);
  return WRS_OK;
}

int wrs_kv_ensure_slots(wrs_kv* kv, size_t n_slots) {
  if (!kv) return WRS_EINVAL;
  wrs_attn_ctx* c = kv->ctx;
  std::lock_guard<std::mutex> lk(c->mu);
  if (n_slots <= kv->n_slots) return WRS_OK;
  if (!fits_int(n_slots)) return fail(c, WRS_EINVAL, "n_slots exceeds 2^31");
  DeviceGuard g(c->device);
  const size_t slot_bytes = kv->n_heads * kv->plane() * kv->esize();
  const size_t bytes = kv->n_layers * n_slots * slot_bytes;
  void *nk = nullptr, *nv = nullptr;
  if (hipMalloc(&nk, bytes) != hipSuccess || hipMalloc(&nv, bytes) != hipSuccess) {
    if (nk) (void)hipFree(nk);
    return fail(c, WRS_ENOMEM, "wrs_kv_ensure_slots: hipMalloc failed");
  }
  if (kv->n_slots) {
    const size_t w = kv->n_slots * slot_bytes;
    WRS_HIP(c, hipMemcpy2DAsync(nk, n_slots * slot_bytes, kv->k_self, w, w, kv->n_layers,
                                hipMemcpyDeviceToDevice, c->stream));
    WRS_HIP(c, hipMemcpy2DAsync(nv, n_slots * slot_bytes, kv->v_self, w, w, kv->n_layers,
                                hipMemcpyDeviceToDevice, c->stream));
    WRS_HIP(c, hipStreamSynchronize(c->stream));
    (void)hipFree(kv->k_self);
    (void)hipFree(kv->v_self);
  }
  kv->k_self = nk;
  kv->v_self = nv;
  kv->n_slots = n_slots;
  kv->len.resize(n_slots, 0);
  return WRS_OK;
}

int wrs_kv_copy_slot(wrs_kv* kv, size_t dst, size_t src) {
  if (!kv) return WRS_EINVAL;
  wrs_attn_ctx* c = kv->ctx;
  std::lock_guard<std::mutex> lk(c->mu);
  if (dst >= kv->n_slots || src >= kv->n_slots) return fail(c, WRS_ERANGE, "slot out of range");
  if (dst == src) return WRS_OK;
  DeviceGuard g(c->device);
  // Strides and row counts in f16-sized rows (twice the rows for f32 planes).
  const size_t w = kv->word_scale();
  const int64_t layer_stride =
      static_cast<int64_t>(kv->n_slots * kv->n_heads * kv->plane() * w);
  const int64_t plane = static_cast<int64_t>(kv->plane() * w);
  const int n = static_cast<int>(kv->len[src] * w);
  WRS_HIP(c, wrs::launch_kv_copy_planes(kv->words(kv->k_self, kv->self_off(0, src)),
                                        kv->words(kv->k_self, kv->self_off(0, dst)), layer_stride,
                                        plane, static_cast<int>(kv->n_layers),
                                        static_cast<int>(kv->n_heads), n, c->stream));
  WRS_HIP(c, wrs::launch_kv_copy_planes(kv->words(kv->v_self, kv->self_off(0, src)),
                                        kv->words(kv->v_self, kv->self_off(0, dst)), layer_stride,
                                        plane, static_cast<int>(kv->n_layers),
                                        static_cast<int>(kv->n_heads), n, c->stream));
  kv->len[dst] = kv->len[src];
  return WRS_OK;
}

int wrs_kv_slot_len(wrs_kv* kv, size_t slot, size_t* len) {
  if (!kv || !len) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  if (slot >= kv->n_slots) return fail(kv->ctx, WRS_ERANGE, "slot out of range");
  *len = kv->len[slot];
  return WRS_OK;
}

int wrs_kv_set_len(wrs_kv* kv, size_t slot, size_t len) {
  if (!kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  if (slot >= kv->n_slots) return fail(kv->ctx, WRS_ERANGE, "slot out of range");
  if (len > kv->len[slot])
    return fail(kv->ctx, WRS_EINVAL, "set_len: rows beyond the stored history do not exist");
  kv->len[slot] = len;
  return WRS_OK;
}

int wrs_kv_slide_to_fit(wrs_kv* kv, size_t slot, size_t n_new, size_t max_ctx, size_t* pos) {
  if (!kv) return WRS_EINVAL;
  wrs_attn_ctx* c = kv->ctx;
  std::lock_guard<std::mutex> lk(c->mu);
  if (slot >= kv->n_slots) return fail(c, WRS_ERANGE, "slot out of range");
  size_t t_past = kv->len[slot];
  if (t_past + n_new > max_ctx) {  // decoder.rs:250-261
    const size_t drop = std::min(t_past + n_new - max_ctx, t_past);
    DeviceGuard g(c->device);
    // In f16-sized rows: an f32 row moves as two.
    const size_t w = kv->word_scale();
    const int64_t layer_stride =
        static_cast<int64_t>(kv->n_slots * kv->n_heads * kv->plane() * w);
    const int64_t plane = static_cast<int64_t>(kv->plane() * w);
    for (void* base : {kv->k_self, kv->v_self})
      WRS_HIP(c, wrs::launch_kv_slide(kv->words(base, kv->self_off(0, slot)), layer_stride, plane,
                                      static_cast<int>(kv->n_layers),
                                      static_cast<int>(kv->n_heads), static_cast<int>(t_past * w),
                                      static_cast<int>(drop * w), c->stream));
    t_past -= drop;
    kv->len[slot] = t_past;
  }
  if (pos) *pos = t_past;
  return WRS_OK;
}

int wrs_kv_append(wrs_kv* kv, size_t layer, size_t slot, const float* k_rows,
                  const float* v_rows, size_t n, int src_on_host) {
  if (!kv) return WRS_EINVAL;
  wrs_attn_ctx* c = kv->ctx;
  std::lock_guard<std::mutex> lk(c->mu);
  if (layer >= kv->n_layers || slot >= kv->n_slots) return fail(c, WRS_ERANGE, "layer/slot out of range");
  if (n == 0) return WRS_OK;
  if (!k_rows || !v_rows) return fail(c, WRS_EINVAL, "null rows");
  const size_t pos = kv->len[slot];
  if (pos + n > kv->max_ctx) return fail(c, WRS_ERANGE, "append past the arena's max_ctx");
  DeviceGuard g(c->device);
  const size_t floats = n * kv->d_model();
  int rc = WRS_OK;
  if (src_on_host) {
    rc = grow(c, &c->stage, &c->stage_bytes, 2 * align_up(floats * 4, 256), false);
    if (rc) return rc;
  }
  const float* dk = to_device_f32(c, k_rows, floats, src_on_host, 0, &rc);
  if (rc) return rc;
  const float* dv = to_device_f32(c, v_rows, floats, src_on_host, align_up(floats * 4, 256), &rc);
  if (rc) return rc;
  const int64_t dm = static_cast<int64_t>(kv->d_model());
  const int64_t plane = static_cast<int64_t>(kv->plane());
  const size_t off = kv->self_off(layer, slot);
  rc = write_rows(c, kv, dk, dm, n, kv->k_self, off, plane, pos);
  if (rc) return rc;
  rc = write_rows(c, kv, dv, dm, n, kv->v_self, off, plane, pos);
  if (rc) return rc;
  if (src_on_host) WRS_HIP(c, hipStreamSynchronize(c->stream));
  return WRS_OK;
}

int wrs_kv_advance(wrs_kv* kv, size_t slot, size_t n) {
  if (!kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  if (slot >= kv->n_slots) return fail(kv->ctx, WRS_ERANGE, "slot out of range");
  if (kv->len[slot] + n > kv->max_ctx) return fail(kv->ctx, WRS_ERANGE, "advance past max_ctx");
  kv->len[slot] += n;
  return WRS_OK;
}

int wrs_kv_set_cross(wrs_kv* kv, size_t layer, const float* k, const float* v, size_t n_audio,
                     int src_on_host) {
  if (!kv) return WRS_EINVAL;
  wrs_attn_ctx* c = kv->ctx;
  std::lock_guard<std::mutex> lk(c->mu);
  if (layer >= kv->n_layers) return fail(c, WRS_ERANGE, "layer out of range");
  if (n_audio > kv->n_audio_max) return fail(c, WRS_ERANGE, "n_audio exceeds the arena");
  if (n_audio && (!k || !v)) return fail(c, WRS_EINVAL, "null rows");
  DeviceGuard g(c->device);
  const size_t floats = n_audio * kv->d_model();
  int rc = WRS_OK;
  if (src_on_host && floats) {
    rc = grow(c, &c->stage, &c->stage_bytes, 2 * align_up(floats * 4, 256), false);
    if (rc) return rc;
  }
  if (floats) {
    const float* dk = to_device_f32(c, k, floats, src_on_host, 0, &rc);
    if (rc) return rc;
    const float* dv = to_device_f32(c, v, floats, src_on_host, align_up(floats * 4, 256), &rc);
    if (rc) return rc;
    const int64_t dm = static_cast<int64_t>(kv->d_model());
    const int64_t plane = static_cast<int64_t>(kv->n_audio_max * 64);
    rc = write_rows(c, kv, dk, dm, n_audio, kv->k_cross, kv->cross_off(layer), plane, 0);
    if (rc) return rc;
    rc = write_rows(c, kv, dv, dm, n_audio, kv->v_cross, kv->cross_off(layer), plane, 0);
    if (rc) return rc;
    if (src_on_host) WRS_HIP(c, hipStreamSynchronize(c->stream));
  }
  kv->cross_len[layer] = n_audio;
  return WRS_OK;
}

int wrs_kv_cross_len(wrs_kv* kv, size_t layer, size_t* n_audio) {
  if (!kv || !n_audio) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  if (layer >= kv->n_layers) return fail(kv->ctx, WRS_ERANGE, "layer out of range");
  *n_audio = kv->cross_len[layer];
  return WRS_OK;
}

int wrs_kv_self_planes(wrs_kv* kv, void** k, void** v, size_t* slot_stride_elems) {
  if (!kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  if (k) *k = kv->k_self;
  if (v) *v = kv->v_self;
  if (slot_stride_elems) *slot_stride_elems = kv->n_heads * kv->plane();
  return WRS_OK;
}

int wrs_kv_cross_planes(wrs_kv* kv, void** k, void** v) {
  if (!kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(kv->ctx->mu);
  if (k) *k = kv->k_cross;
  if (v) *v = kv->v_cross;
  return WRS_OK;
}

int wrs_attn_decode_self(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const size_t* slots,
                         size_t n, const float* q, float* out) {
  if (!c || !kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (layer >= kv->n_layers) return fail(c, WRS_ERANGE, "layer out of range");
  if (n == 0) return WRS_OK;
  if (!slots || !q || !out) return fail(c, WRS_EINVAL, "null argument");
  DeviceGuard g(c->device);
  const int64_t dm = static_cast<int64_t>(kv->d_model());
  for (size_t i0 = 0; i0 < n; i0 += wrs::kMaxDecodeGroups) {
    const size_t m = std::min<size_t>(wrs::kMaxDecodeGroups, n - i0);
    std::vector<int64_t> goff(m);
    std::vector<int> lens(m);
    for (size_t i = 0; i < m; ++i) {
      const size_t s = slots[i0 + i];
      if (s >= kv->n_slots) return fail(c, WRS_ERANGE, "slot out of range");
      // The step's own row sits at position len (appended, not yet advanced).
      if (kv->len[s] + 1 > kv->max_ctx) return fail(c, WRS_ERANGE, "slot is full");
      goff[i] = static_cast<int64_t>(kv->self_off(layer, s));
      lens[i] = static_cast<int>(kv->len[s] + 1);
    }
    int rc = kv->f32()
                 ? exact_arena(c, kv, q + i0 * dm, out + i0 * dm, kv->k_self, kv->v_self,
                               static_cast<int64_t>(kv->plane()), goff, lens, 1, 0,
                               static_cast<int>(m))
                 : decode_impl(c, q + i0 * dm, dm, out + i0 * dm, dm, wrs_kv::u16(kv->k_self),
                               wrs_kv::u16(kv->v_self), static_cast<int64_t>(kv->plane()), goff,
                               lens, 1, static_cast<int>(kv->n_heads));
    if (rc) return rc;
  }
  return WRS_OK;
}

}  // extern "C"

namespace {

int decode_cross_impl(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q,
                      size_t n_beams, float* out, unsigned char* fixed) {
  if (layer >= kv->n_layers) return fail(c, WRS_ERANGE, "layer out of range");
  if (n_beams == 0) return WRS_OK;
  if (!q || !out) return fail(c, WRS_EINVAL, "null argument");
  if (reinterpret_cast<uintptr_t>(q) & 15)
    return fail(c, WRS_EINVAL, "q must be 16-byte aligned");
  DeviceGuard g(c->device);
  const int64_t dm = static_cast<int64_t>(kv->d_model());
  const size_t L = kv->cross_len[layer];
  if (L == 0) {
    // attention.rs:93-96: no keys, zero output (the plane may not exist).
    WRS_HIP(c, wrs::launch_fill_zero_rows(out, 0, 0, dm, 1, 1, static_cast<int>(n_beams),
                                          static_cast<int>(dm), c->stream));
    return WRS_OK;
  }
  if (kv->f32()) {
    // f32 arena: every beam row on the exact kernel (attention.rs:246-434,
    // the single-token path each beam's decoder call takes).
    if (fixed) return fail(c, WRS_EUNSUPPORTED, "allocation-free decode needs an f16 arena");
    constexpr size_t kRows = 4096;
    for (size_t b0 = 0; b0 < n_beams; b0 += kRows) {
      const int rows = static_cast<int>(std::min(kRows, n_beams - b0));
      int rc = exact_arena(c, kv, q + b0 * dm, out + b0 * dm, kv->k_cross, kv->v_cross,
                           static_cast<int64_t>(kv->n_audio_max * 64),
                           {static_cast<int64_t>(kv->cross_off(layer))}, {static_cast<int>(L)},
                           rows, 0, rows);
      if (rc) return rc;
    }
    return WRS_OK;
  }
  // All beams of the utterance share one read of the plane; beyond 8 beams the
  // rows go in further launches of up to 8 (which reuse the same scratch in
  // stream order).
  for (size_t b0 = 0; b0 < n_beams; b0 += wrs::kMaxRowsPerGroup) {
    const size_t rows = std::min<size_t>(wrs::kMaxRowsPerGroup, n_beams - b0);
    std::vector<int64_t> goff(1, static_cast<int64_t>(kv->cross_off(layer)));
    std::vector<int> lens(1, static_cast<int>(L));
    int rc = decode_impl(c, q + b0 * dm, dm, out + b0 * dm, dm, wrs_kv::u16(kv->k_cross),
                         wrs_kv::u16(kv->v_cross), static_cast<int64_t>(kv->n_audio_max * 64),
                         goff, lens, static_cast<int>(rows), static_cast<int>(kv->n_heads), fixed);
    if (rc) return rc;
  }
  return WRS_OK;
}

// Cross-attention of n query rows over one layer's plane on the split-K decode
// kernel: groups of kMaxRowsPerGroup rows share each read of the plane, up to
// kMaxDecodeGroups groups per launch, and the remaining rows one last group.
// With lse, the rows' statistics too ([head][n][2], exp2 domain).
int cross_rows_impl(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q, size_t n,
                    float* out, float* lse) {
  if (layer >= kv->n_layers) return fail(c, WRS_ERANGE, "layer out of range");
  if (n == 0) return WRS_OK;
  if (!q || !out) return fail(c, WRS_EINVAL, "null argument");
  if (reinterpret_cast<uintptr_t>(q) & 15)
    return fail(c, WRS_EINVAL, "q must be 16-byte aligned");
  if (!fits_int(n)) return fail(c, WRS_EINVAL, "dimension exceeds 2^31");
  DeviceGuard g(c->device);
  const int64_t dm = static_cast<int64_t>(kv->d_model());
  const size_t L = kv->cross_len[layer];
  if (L == 0) {
    // attention.rs:93-96: no keys, zero output (the plane may not exist).
    WRS_HIP(c, wrs::launch_fill_zero_rows(out, 0, 0, dm, 1, 1, static_cast<int>(n),
                                          static_cast<int>(dm), c->stream));
    return WRS_OK;
  }
  if (kv->f32()) {
    // f32 arena: the prompt rows as flash_attention_2 takes them
    // (attention.rs:79-105): one row on the exact single-token kernel, more on
    // the f32 prefill kernel. No row statistics on this path.
    if (lse) return fail(c, WRS_EUNSUPPORTED, "row statistics need an f16 arena");
    const int64_t plane = static_cast<int64_t>(kv->n_audio_max * 64);
    if (n == 1)
      return exact_arena(c, kv, q, out, kv->k_cross, kv->v_cross, plane,
                         {static_cast<int64_t>(kv->cross_off(layer))}, {static_cast<int>(L)}, 1,
                         0, 1);
    const wrs_layout lq{0, 64, dm};
    const wrs_layout lkv{0, plane, 64};
    return prefill_impl(c, WRS_F32, q, lq, WRS_F32, wrs_kv::f32p(kv->k_cross, kv->cross_off(layer)),
                        lkv, wrs_kv::f32p(kv->v_cross, kv->cross_off(layer)), lkv, out, lq, 1,
                        kv->n_heads, n, L, 64, 0, 0);
  }
  for (size_t r0 = 0; r0 < n;) {
    const size_t left = n - r0;
    const int rpg = static_cast<int>(std::min<size_t>(left, wrs::kMaxRowsPerGroup));
    const size_t groups =
        left >= static_cast<size_t>(wrs::kMaxRowsPerGroup)
            ? std::min<size_t>(left / wrs::kMaxRowsPerGroup, wrs::kMaxDecodeGroups)
            : 1;
    std::vector<int64_t> goff(groups, static_cast<int64_t>(kv->cross_off(layer)));
    std::vector<int> lens(groups, static_cast<int>(L));
    int rc = decode_impl(c, q + r0 * dm, dm, out + r0 * dm, dm, wrs_kv::u16(kv->k_cross),
                         wrs_kv::u16(kv->v_cross), static_cast<int64_t>(kv->n_audio_max * 64),
                         goff, lens, rpg,
                         static_cast<int>(kv->n_heads), nullptr, lse, static_cast<int>(n),
                         static_cast<int>(r0));
    if (rc) return rc;
    r0 += groups * static_cast<size_t>(rpg);
  }
  return WRS_OK;
}

}  // namespace

extern "C" {

int wrs_attn_decode_cross(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q,
                          size_t n_beams, float* out) {
  if (!c || !kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  return decode_cross_impl(c, kv, layer, q, n_beams, out, nullptr);
}

int wrs_attn_decode_cross_noalloc(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q,
                                  size_t n_beams, float* out) {
  if (!c || !kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (kv->f32()) return fail(c, WRS_EUNSUPPORTED, "allocation-free decode needs an f16 arena");
  int rc = WRS_OK;
  unsigned char* fixed = noalloc_slot_ptr(c, &rc);
  if (!fixed) return rc;
  return decode_cross_impl(c, kv, layer, q, n_beams, out, fixed);
}

int wrs_attn_prefill_self(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, size_t slot, const float* q,
                          size_t n_tokens, float* out) {
  if (!c || !kv) return WRS_EINVAL;
  if (n_tokens == 1) return wrs_attn_decode_self(c, kv, layer, &slot, 1, q, out);
  std::lock_guard<std::mutex> lk(c->mu);
  if (layer >= kv->n_layers || slot >= kv->n_slots) return fail(c, WRS_ERANGE, "layer/slot out of range");
  if (n_tokens == 0) return WRS_OK;
  const size_t t_past = kv->len[slot];
  if (t_past + n_tokens > kv->max_ctx) return fail(c, WRS_ERANGE, "rows past max_ctx");
  DeviceGuard g(c->device);
  const int64_t dm = static_cast<int64_t>(kv->d_model());
  if (kv->f32()) {
    // f32 arena: mha_with_cache's multi-token path (decoder.rs:857-892) on the
    // exact kernel; prompt row i sees t_past + 1 + i keys.
    constexpr size_t kRows = 4096;
    for (size_t r0 = 0; r0 < n_tokens; r0 += kRows) {
      const int rows = static_cast<int>(std::min(kRows, n_tokens - r0));
      int rc = exact_arena(c, kv, q + r0 * dm, out + r0 * dm, kv->k_self, kv->v_self,
                           static_cast<int64_t>(kv->plane()),
                           {static_cast<int64_t>(kv->self_off(layer, slot))},
                           {static_cast<int>(t_past + 1 + r0)}, rows, 1, rows);
      if (rc) return rc;
    }
    return WRS_OK;
  }
  const wrs_layout lq{0, 64, dm};
  const wrs_layout lkv{0, static_cast<int64_t>(kv->plane()), 64};
  const uint16_t* kb = wrs_kv::u16(kv->k_self, kv->self_off(layer, slot));
  const uint16_t* vb = wrs_kv::u16(kv->v_self, kv->self_off(layer, slot));
  return prefill_impl(c, WRS_F32, q, lq, WRS_F16, kb, lkv, vb, lkv, out, lq, 1, kv->n_heads,
                      n_tokens, t_past + n_tokens, 64, 1, t_past);
}

int wrs_attn_prefill_cross(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q,
                           size_t n_tokens, float* out) {
  if (!c || !kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  return cross_rows_impl(c, kv, layer, q, n_tokens, out, nullptr);
}

int wrs_attn_prefill_cross_lse(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q,
                               size_t n_tokens, float* out, float* lse) {
  if (!c || !kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (!lse && n_tokens) return fail(c, WRS_EINVAL, "null lse");
  return cross_rows_impl(c, kv, layer, q, n_tokens, out, lse);
}

}  // extern "C"

namespace {

int capture_impl(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q, size_t n_tokens,
                 const size_t* slots, const size_t* heads, size_t n_pairs, size_t n_selected,
                 size_t row_offset, float* out, size_t out_len, const float* lse) {
  if (!c || !kv) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (layer >= kv->n_layers) return fail(c, WRS_ERANGE, "layer out of range");
  if (n_tokens == 0 || n_pairs == 0) return WRS_OK;
  if (!q || !out || !slots || !heads) return fail(c, WRS_EINVAL, "null argument");
  for (size_t p = 0; p < n_pairs; ++p) {
    // decoder.rs:814-816 slices q/k at head * d_head (panics past d_model);
    // the slot comes from enumerating the caller's head list (decoder.rs:683).
    if (heads[p] >= kv->n_heads) return fail(c, WRS_EINVAL, "head index >= n_heads");
    if (slots[p] >= n_selected) return fail(c, WRS_EINVAL, "slot index >= n_selected");
  }
  const size_t n_audio = kv->cross_len[layer];
  // decoder.rs:812 / :822: out holds (row_offset + n_tokens) rows of
  // n_selected * n_audio weights.
  if (out_len / std::max<size_t>(1, n_selected * n_audio) < row_offset + n_tokens &&
      n_audio > 0)
    return fail(c, WRS_EINVAL, "out shorter than (row_offset + n_tokens) * n_selected * n_audio");
  if (n_audio == 0) return WRS_OK;  // softmax of an empty row (softmax.rs:2-4)
  if ((reinterpret_cast<uintptr_t>(q) & 15) != 0)
    return fail(c, WRS_EINVAL, "q must be 16-byte aligned");
  if (n_tokens > static_cast<size_t>(65535) * wrs::kCaptureRows ||
      (row_offset + n_tokens) * n_selected > static_cast<size_t>(INT32_MAX))
    return fail(c, WRS_EINVAL, "capture shape too large");
  DeviceGuard g(c->device);
  wrs::CaptureArgs a{};
  a.q = q;
  a.out = out;
  a.q_rs = static_cast<int64_t>(kv->d_model());
  a.kv_hs = static_cast<int64_t>(kv->n_audio_max * 64);
  a.n_tokens = static_cast<int>(n_tokens);
  a.n_audio = static_cast<int>(n_audio);
  a.n_selected = static_cast<int>(n_selected);
  a.row_offset = static_cast<int>(row_offset);
  a.scale_log2 = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) (decoder.rs:810) * log2(e)
  a.lse = lse;
  if (kv->f32()) {
    // f32 planes: scores and softmax as decoder.rs:814-825 computes them, one
    // workgroup per (row, pair); row statistics are not used.
    if (lse) return fail(c, WRS_EUNSUPPORTED, "row statistics need an f16 arena");
    a.k32 = wrs_kv::f32p(kv->k_cross, kv->cross_off(layer));
    a.scale = 0.125f;  // 1/sqrt(64) (decoder.rs:810)
    for (size_t p0 = 0; p0 < n_pairs; p0 += wrs::kMaxCapturePairs) {
      const size_t np = std::min<size_t>(wrs::kMaxCapturePairs, n_pairs - p0);
      a.n_pairs = static_cast<int>(np);
      for (size_t p = 0; p < np; ++p) {
        a.slot[p] = static_cast<int>(slots[p0 + p]);
        a.head[p] = static_cast<int>(heads[p0 + p]);
      }
      WRS_HIP(c, wrs::launch_capture_cross_f32(a, c->stream));
    }
    return WRS_OK;
  }
  a.k = reinterpret_cast<const _Float16*>(wrs_kv::u16(kv->k_cross, kv->cross_off(layer)));
  if (!lse) {  // two passes: chunk statistics in the context
    const size_t pb =
        wrs::capture_part_floats(static_cast<int>(std::min<size_t>(n_pairs, wrs::kMaxCapturePairs)),
                                 a.n_tokens, a.n_audio) * sizeof(float);
    int rc = grow(c, reinterpret_cast<void**>(&c->cap_part), &c->cap_part_bytes, pb, false);
    if (rc) return rc;
    a.part = c->cap_part;
  }
  for (size_t p0 = 0; p0 < n_pairs; p0 += wrs::kMaxCapturePairs) {
    const size_t np = std::min<size_t>(wrs::kMaxCapturePairs, n_pairs - p0);
    a.n_pairs = static_cast<int>(np);
    for (size_t p = 0; p < np; ++p) {
      a.slot[p] = static_cast<int>(slots[p0 + p]);
      a.head[p] = static_cast<int>(heads[p0 + p]);
    }
    WRS_HIP(c, wrs::launch_capture_cross_f16(a, c->stream));
  }
  return WRS_OK;
}

}  // namespace

extern "C" {

int wrs_attn_capture_cross_heads(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q,
                                 size_t n_tokens, const size_t* slots, const size_t* heads,
                                 size_t n_pairs, size_t n_selected, size_t row_offset, float* out,
                                 size_t out_len) {
  return capture_impl(c, kv, layer, q, n_tokens, slots, heads, n_pairs, n_selected, row_offset,
                      out, out_len, nullptr);
}

int wrs_attn_capture_cross_heads_lse(wrs_attn_ctx* c, wrs_kv* kv, size_t layer, const float* q,
                                     size_t n_tokens, const size_t* slots, const size_t* heads,
                                     size_t n_pairs, size_t n_selected, size_t row_offset,
                                     float* out, size_t out_len, const float* lse) {
  if (!lse) {
    if (!c) return WRS_EINVAL;
    std::lock_guard<std::mutex> lk(c->mu);
    return fail(c, WRS_EINVAL, "null lse");
  }
  return capture_impl(c, kv, layer, q, n_tokens, slots, heads, n_pairs, n_selected, row_offset,
                      out, out_len, lse);
}

}  // extern "C"

namespace {

// Shared front half of the projection entry points: validates x and the
// shape, splits f32 rows into the context scratch, and fills the x part of
// the launch arguments. Caller holds c->mu and the device guard.
int linear_prepare(wrs_attn_ctx* c, int x_dtype, const void* x, int64_t x_rs, size_t n_tokens,
                   size_t n_in, size_t n_out, wrs::LinearArgs& a) {
  if (n_in == 0 || n_in % wrs::kLinearK != 0)
    return fail(c, WRS_EUNSUPPORTED, "n_in must be a positive multiple of 64");
  if (n_out % 4 != 0) return fail(c, WRS_EUNSUPPORTED, "n_out must be a multiple of 4");
  if (n_tokens > static_cast<size_t>(INT32_MAX / 2) || n_in > (1u << 20) ||
      n_out > static_cast<size_t>(INT32_MAX / 2))
    return fail(c, WRS_EINVAL, "projection shape too large");
  if (x_rs < static_cast<int64_t>(n_in)) return fail(c, WRS_EINVAL, "x row stride < n_in");
  // The kernel addresses W and x through buffer resources: 32-bit byte
  // offsets, including the rows past the edge of the last tile.
  const int64_t xs_rs = x_dtype == WRS_F32 ? wrs::kSplitParts * static_cast<int64_t>(n_in) : x_rs;
  if ((static_cast<int64_t>(n_tokens) + 256) * xs_rs * 2 >= (int64_t{1} << 31) ||
      (static_cast<int64_t>(n_out) + 256) * static_cast<int64_t>(n_in) * 2 >= (int64_t{1} << 31))
    return fail(c, WRS_EUNSUPPORTED, "x or W span beyond the kernel's 2 GiB addressing");
  a.n_tokens = static_cast<int>(n_tokens);
  a.n_in = static_cast<int>(n_in);
  a.n_out = static_cast<int>(n_out);
  if (x_dtype == WRS_F16) {
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (x_rs % 8))
      return fail(c, WRS_EUNSUPPORTED, "f16 x rows must be 16-byte aligned");
    a.x = static_cast<const _Float16*>(x);
    a.x_rs = x_rs;
    a.row_scale = nullptr;
    a.k_total = a.n_in;
    return WRS_OK;
  }
  if (x_dtype != WRS_F32) return fail(c, WRS_EUNSUPPORTED, "x must be f32 or f16");
  const size_t split_bytes = align_up(n_tokens * wrs::kSplitParts * n_in * 2, 256);
  int rc = grow(c, &c->lin_x, &c->lin_x_bytes, split_bytes + n_tokens * 4, false);
  if (rc) return rc;
  auto* xs = static_cast<_Float16*>(c->lin_x);
  auto* scale = reinterpret_cast<float*>(static_cast<char*>(c->lin_x) + split_bytes);
  WRS_HIP(c, wrs::launch_linear_split(static_cast<const float*>(x), x_rs, a.n_tokens, a.n_in, xs,
                                      scale, c->stream));
  a.x = xs;
  a.x_rs = wrs::kSplitParts * static_cast<int64_t>(n_in);
  a.row_scale = scale;
  a.k_total = wrs::kSplitParts * a.n_in;
  return WRS_OK;
}

bool aligned_out(const void* p, int dt, int64_t rs, int64_t hs) {
  const uintptr_t need = dt == WRS_F32 ? 16 : 8;
  return (reinterpret_cast<uintptr_t>(p) % need) == 0 && rs % 4 == 0 && hs % 4 == 0;
}

// W_g x + bias_g for g < n_groups weight matrices of one shape against one
// input, in one launch (the caller holds c->mu). bias may be NULL, or hold
// NULL entries.
int linear_impl(wrs_attn_ctx* c, int x_dtype, const void* x, size_t x_len, int64_t x_row_stride,
                int n_groups, const void* const* w, const float* const* bias, size_t n_tokens,
                size_t n_in, size_t n_out, int out_dtype, void* const* out,
                const size_t* out_len, int64_t out_row_stride, int64_t out_head_stride,
                const float* ln_g = nullptr, const float* ln_b = nullptr, float ln_eps = 0.f,
                int act = wrs::kActNone) {
  if (n_tokens == 0 || n_out == 0) return WRS_OK;  // quant.rs:430-432
  if (!x) return fail(c, WRS_EINVAL, "null argument");
  for (int gi = 0; gi < n_groups; ++gi)
    if (!w[gi] || !out[gi]) return fail(c, WRS_EINVAL, "null argument");
  // quant.rs:424-425: x holds num_tokens rows of cols, output num_tokens * rows
  if (x_row_stride < 0 || out_row_stride < 0 || out_head_stride < 0)
    return fail(c, WRS_EINVAL, "negative stride");
  if (x_len < (n_tokens - 1) * static_cast<size_t>(x_row_stride) + n_in)
    return fail(c, WRS_EINVAL, "x shorter than n_tokens rows of n_in");
  const size_t last_g = (n_out - 1) / 64;
  const size_t max_off =
      (n_tokens - 1) * static_cast<size_t>(out_row_stride) +
      std::max(last_g * static_cast<size_t>(out_head_stride) + (n_out - 1) % 64,
               last_g ? (last_g - 1) * static_cast<size_t>(out_head_stride) + 63 : 0);
  for (int gi = 0; gi < n_groups; ++gi)
    if (out_len[gi] <= max_off) return fail(c, WRS_EINVAL, "out shorter than the written range");
  if (out_dtype != WRS_F32 && out_dtype != WRS_F16 && out_dtype != WRS_BF16)
    return fail(c, WRS_EINVAL, "unknown output dtype");
  for (int gi = 0; gi < n_groups; ++gi)
    if (reinterpret_cast<uintptr_t>(w[gi]) & 15)
      return fail(c, WRS_EUNSUPPORTED, "w needs 16-byte alignment");
  DeviceGuard g(c->device);
  if (n_tokens <= static_cast<size_t>(wrs::kGemvMaxRows) &&
      n_tokens * n_in <= static_cast<size_t>(wrs::kGemvXFloats)) {
    // Decode-sized batch: the f16 weight stream (f16_gemv_parallel, quant.rs:392-413);
    // any n_out, element-wise stores.
    if (n_in == 0 || n_in % wrs::kLinearK != 0)
      return fail(c, WRS_EUNSUPPORTED, "n_in must be a positive multiple of 64");
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (x_row_stride % (x_dtype == WRS_F32 ? 4 : 8)))
      return fail(c, WRS_EUNSUPPORTED, "x rows must be 16-byte aligned");
    if (x_dtype != WRS_F32 && x_dtype != WRS_F16)
      return fail(c, WRS_EUNSUPPORTED, "x must be f32 or f16");
    if (x_row_stride < static_cast<int64_t>(n_in) || n_in > (1u << 24) ||
        n_out > static_cast<size_t>(INT32_MAX / 2))
      return fail(c, WRS_EINVAL, "projection shape");
    wrs::GemvArgs gv{};
    gv.x = x;
    gv.x_rs = x_row_stride;
    gv.n_tokens = static_cast<int>(n_tokens);
    gv.n_in = static_cast<int>(n_in);
    gv.n_out = static_cast<int>(n_out);
    gv.n_groups = n_groups;
    gv.out_rs = out_row_stride;
    gv.out_hs = out_head_stride;
    gv.ln_g = ln_g;
    gv.ln_b = ln_b;
    gv.ln_eps = ln_eps;
    gv.act = act;
    for (int gi = 0; gi < n_groups; ++gi) {
      gv.w[gi] = static_cast<const _Float16*>(w[gi]);
      gv.bias[gi] = bias ? bias[gi] : nullptr;
      gv.out[gi] = out[gi];
    }
    WRS_HIP(c, wrs::launch_gemv_f16w(gv, static_cast<wrs::DType>(x_dtype),
                                     static_cast<wrs::DType>(out_dtype), c->stream));
    return WRS_OK;
  }
  for (int gi = 0; gi < n_groups; ++gi)
    if (!aligned_out(out[gi], out_dtype, out_row_stride, out_head_stride) ||
        (bias && bias[gi] && (reinterpret_cast<uintptr_t>(bias[gi]) & 15)))
      return fail(c, WRS_EUNSUPPORTED, "bias needs 16-byte, out 4-element alignment");
  if (ln_g) {
    // Larger batches: the LayerNorm runs as its own launch into scratch rows.
    if (x_row_stride != static_cast<int64_t>(n_in))
      return fail(c, WRS_EUNSUPPORTED, "a fused layer norm over more than 8 rows needs packed x rows");
    int rc = grow(c, reinterpret_cast<void**>(&c->ln_x), &c->ln_x_bytes,
                  n_tokens * n_in * sizeof(float), false);
    if (rc) return rc;
    WRS_HIP(c, wrs::launch_layer_norm(static_cast<const float*>(x), ln_g, ln_b, ln_eps,
                                      static_cast<int>(n_tokens), static_cast<int>(n_in),
                                      wrs::kF32, c->ln_x, c->stream));
    x = c->ln_x;
    x_row_stride = static_cast<int64_t>(n_in);
  }
  wrs::LinearArgs a{};
  int rc = linear_prepare(c, x_dtype, x, x_row_stride, n_tokens, n_in, n_out, a);
  if (rc) return rc;
  a.act = act;
  a.n_groups = n_groups;
  a.out_rs = out_row_stride;
  a.out_hs = out_head_stride;
  for (int gi = 0; gi < n_groups; ++gi) {
    a.w[gi] = static_cast<const _Float16*>(w[gi]);
    a.bias[gi] = bias ? bias[gi] : nullptr;
    a.out[gi] = out[gi];
  }
  WRS_HIP(c, wrs::launch_linear_f16w(a, static_cast<wrs::DType>(out_dtype), c->stream));
  return WRS_OK;
}


}  // namespace

extern "C" {

int wrs_linear(wrs_attn_ctx* c, int x_dtype, const void* x, size_t x_len, int64_t x_row_stride,
               const void* w, const float* bias, size_t n_tokens, size_t n_in, size_t n_out,
               int out_dtype, void* out, size_t out_len, int64_t out_row_stride,
               int64_t out_head_stride) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  return linear_impl(c, x_dtype, x, x_len, x_row_stride, 1, &w, &bias, n_tokens, n_in, n_out,
                     out_dtype, &out, &out_len, out_row_stride, out_head_stride);
}

int wrs_linear_group(wrs_attn_ctx* c, int x_dtype, const void* x, size_t x_len,
                     int64_t x_row_stride, size_t n_groups, const void* const* w,
                     const float* const* bias, size_t n_tokens, size_t n_in, size_t n_out,
                     int out_dtype, void* const* out, const size_t* out_len,
                     int64_t out_row_stride, int64_t out_head_stride) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (n_groups == 0 || n_tokens == 0 || n_out == 0) return WRS_OK;
  if (!w || !out || !out_len) return fail(c, WRS_EINVAL, "null argument");
  if (n_groups > static_cast<size_t>(wrs::kMaxLinearGroups))
    return fail(c, WRS_EINVAL, "more weight matrices than one launch takes");
  return linear_impl(c, x_dtype, x, x_len, x_row_stride, static_cast<int>(n_groups), w, bias,
                     n_tokens, n_in, n_out, out_dtype, out, out_len, out_row_stride,
                     out_head_stride);
}

int wrs_linear_fused(wrs_attn_ctx* c, const float* x, size_t x_len, int64_t x_row_stride,
                     const float* ln_gamma, const float* ln_beta, float ln_eps, size_t n_groups,
                     const void* const* w, const float* const* bias, size_t n_tokens,
                     size_t n_in, size_t n_out, int activation, int out_dtype, void* const* out,
                     const size_t* out_len, int64_t out_row_stride, int64_t out_head_stride) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (n_groups == 0 || n_tokens == 0 || n_out == 0) return WRS_OK;
  if (!w || !out || !out_len) return fail(c, WRS_EINVAL, "null argument");
  if (n_groups > static_cast<size_t>(wrs::kMaxLinearGroups))
    return fail(c, WRS_EINVAL, "more weight matrices than one launch takes");
  if ((ln_gamma == nullptr) != (ln_beta == nullptr))
    return fail(c, WRS_EINVAL, "layer norm needs both gamma and beta");
  if (activation != WRS_ACT_NONE && activation != WRS_ACT_GELU)
    return fail(c, WRS_EINVAL, "unknown activation");
  if (ln_gamma && ((reinterpret_cast<uintptr_t>(ln_gamma) & 15) ||
                   (reinterpret_cast<uintptr_t>(ln_beta) & 15)))
    return fail(c, WRS_EUNSUPPORTED, "gamma and beta need 16-byte alignment");
  return linear_impl(c, WRS_F32, x, x_len, x_row_stride, static_cast<int>(n_groups), w, bias,
                     n_tokens, n_in, n_out, out_dtype, out, out_len, out_row_stride,
                     out_head_stride, ln_gamma, ln_beta, ln_eps,
                     activation == WRS_ACT_GELU ? wrs::kActGelu : wrs::kActNone);
}

int wrs_layer_norm(wrs_attn_ctx* c, const float* x, size_t x_len, const float* gamma,
                   const float* beta, float eps, size_t n_tokens, size_t d_model, int out_dtype,
                   void* out, size_t out_len) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  // norm.rs:124-127
  if (x_len != n_tokens * d_model || out_len != n_tokens * d_model)
    return fail(c, WRS_EINVAL, "input/output length != num_tokens * d_model");
  if (n_tokens == 0 || d_model == 0) return WRS_OK;
  if (!x || !gamma || !beta || !out) return fail(c, WRS_EINVAL, "null argument");
  if (out_dtype != WRS_F32 && out_dtype != WRS_F16 && out_dtype != WRS_BF16)
    return fail(c, WRS_EINVAL, "unknown output dtype");
  if (d_model % 4 != 0 || (reinterpret_cast<uintptr_t>(x) & 15) ||
      (reinterpret_cast<uintptr_t>(gamma) & 15) || (reinterpret_cast<uintptr_t>(beta) & 15) ||
      (reinterpret_cast<uintptr_t>(out) & (out_dtype == WRS_F32 ? 15 : 7)))
    return fail(c, WRS_EUNSUPPORTED, "d_model % 4 and 16-byte aligned rows required");
  if (n_tokens > static_cast<size_t>(INT32_MAX) || d_model > static_cast<size_t>(INT32_MAX / 4))
    return fail(c, WRS_EINVAL, "layer_norm shape too large");
  DeviceGuard g(c->device);
  WRS_HIP(c, wrs::launch_layer_norm(x, gamma, beta, eps, static_cast<int>(n_tokens),
                                    static_cast<int>(d_model),
                                    static_cast<wrs::DType>(out_dtype), out, c->stream));
  return WRS_OK;
}

int wrs_gelu_inplace(wrs_attn_ctx* c, float* data, size_t n) {
  if (!c) return WRS_EINVAL;
  std::lock_guard<std::mutex> lk(c->mu);
  if (n == 0) return WRS_OK;
  if (!data) return fail(c, WRS_EINVAL, "null argument");
  if (reinterpret_cast<uintptr_t>(data) & 15)
    return fail(c, WRS_EUNSUPPORTED, "data must be 16-byte aligned");
  DeviceGuard g(c->device);
  WRS_HIP(c, wrs::launch_gelu(data, static_cast<int64_t>(n), c->stream));
  return WRS_OK;
}

int wrs_kv_set_cross_proj(wrs_kv* kv, int x_dtype, const void* enc, size_t enc_len,
                          int64_t enc_row_stride, size_t n_audio, const void* const* w_k,
                          const void* const* w_v, const float* const* b_v) {
  if (!kv) return WRS_EINVAL;
  wrs_attn_ctx* c = kv->ctx;
  std::lock_guard<std::mutex> lk(c->mu);
  if (n_audio > kv->n_audio_max) return fail(c, WRS_ERANGE, "n_audio exceeds the arena");
  if (!w_k || !w_v) return fail(c, WRS_EINVAL, "null weight arrays");
  for (size_t l = 0; l < kv->n_layers; ++l) {
    if (!w_k[l] || !w_v[l]) return fail(c, WRS_EINVAL, "null layer weight");
    if ((reinterpret_cast<uintptr_t>(w_k[l]) & 15) || (reinterpret_cast<uintptr_t>(w_v[l]) & 15) ||
        (b_v && b_v[l] && (reinterpret_cast<uintptr_t>(b_v[l]) & 15)))
      return fail(c, WRS_EUNSUPPORTED, "weights and biases need 16-byte alignment");
  }
  if (n_audio > 0) {
    if (!enc) return fail(c, WRS_EINVAL, "null encoder output");
    if (enc_row_stride < 0 ||
        enc_len < (n_audio - 1) * static_cast<size_t>(enc_row_stride) + kv->d_model())
      return fail(c, WRS_EINVAL, "encoder output shorter than n_audio rows of d_model");
    DeviceGuard g(c->device);
    wrs::LinearArgs a{};
    const size_t dm = kv->d_model();
    int rc = linear_prepare(c, x_dtype, enc, enc_row_stride, n_audio, dm, dm, a);
    if (rc) return rc;
    a.out_rs = 64;  // [head][n_audio_max][64] planes
    a.out_hs = static_cast<int64_t>(kv->n_audio_max * 64);
    // decoder.rs:433-442: K without bias, V with cross_attn_v_b; every layer's
    // K and V in as few launches as the group limit allows.
    const size_t per_launch = wrs::kMaxLinearGroups / 2;
    for (size_t l0 = 0; l0 < kv->n_layers; l0 += per_launch) {
      const size_t nl = std::min(per_launch, kv->n_layers - l0);
      a.n_groups = static_cast<int>(2 * nl);
      for (size_t i = 0; i < nl; ++i) {
        const size_t l = l0 + i;
        a.w[2 * i] = static_cast<const _Float16*>(w_k[l]);
        a.bias[2 * i] = nullptr;
        a.out[2 * i] = kv->words(kv->k_cross, kv->cross_off(l));
        a.w[2 * i + 1] = static_cast<const _Float16*>(w_v[l]);
        a.bias[2 * i + 1] = b_v ? b_v[l] : nullptr;
        a.out[2 * i + 1] = kv->words(kv->v_cross, kv->cross_off(l));
      }
      WRS_HIP(c, wrs::launch_linear_f16w(a, kv->f32() ? wrs::kF32 : wrs::kF16, c->stream));
    }
  }
  for (size_t l = 0; l < kv->n_layers; ++l) kv->cross_len[l] = n_audio;
  return WRS_OK;
}

}  // extern "C"
