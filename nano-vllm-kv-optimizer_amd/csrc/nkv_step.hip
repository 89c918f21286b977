// The sparse decode layer-step for a batch of layers in one host call:
// selection (score + top-k) then attention, with the layers split into
// contiguous ranges enqueued on several streams.
//
// Replaces, for every layer of a model at once, steps 2 and 5 of
// M12LayerRuntime.decode (nanovllm/sparse/m12_runtime.py:1141-1346): the
// selection of _gpu_select (:959-1055) and the attention over
// [selected | sink | recent | new token] (:1212-1320), with the recent-ring
// shift + append of step 1 (:1164-1172) done by the attention launch.
//
// The layers are independent, so each range runs exactly the launches a
// single-range call would make for those layers (same kernels, same launch
// shapes: the attention split count is the caller's), and the results are
// identical.  What the ranges can buy is overlap: one range's launch-bound
// top-k and merge kernels, and every kernel's tail, run beside another
// range's bandwidth-bound scoring and attention.  The per-call joins cost
// GPU time too (on the 36-layer 32K step two ranges measured 135 us against
// 128 us for one), so one range is the default of the Python runtime.
#include <mutex>
#include <vector>

#include "nkv_attend_common.h"

namespace nkv {
namespace {

constexpr int kMaxStepStreams = 8;

// ---- scratch of the allocation-free decode step ---------------------------
// One array per GPU, in the library's code object: the score keys (uint32
// [L][nblocks], zero between calls) then the split partials of the attention.
constexpr int64_t kScratchBytes = int64_t(16) << 20;
constexpr int64_t kScratchKeyBytes = int64_t(1) << 20;
constexpr int64_t kScratchKeys = kScratchKeyBytes / 4;                      // 262144 keys
constexpr int64_t kScratchPartialFloats = (kScratchBytes - kScratchKeyBytes) / 4;
constexpr int kMaxScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The device address of this GPU's `scratch` (the host-side name is only a
// stand-in for the symbol), looked up with the device current until one
// look-up succeeds; that look-up also clears the key region on `s` with a
// fill kernel (every later call leaves the keys it used at zero).  A failed
// set-up leaves the slot empty, so the next call tries again.
__global__ void zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

struct ScratchSlot {
  std::mutex mu;
  void* ptr = nullptr;   // set (under mu) only once the look-up and the clear were enqueued
};
ScratchSlot g_scratch[kMaxScratchDevices];

int scratch_address(hipStream_t s, char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("nkv_decode_step_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return NKV_ERR_HIP;
  }
  NKV_CHECK_SUPPORTED(dev >= 0 && dev < kMaxScratchDevices, "nkv_decode_step_noalloc: device %d beyond %d", dev,
                      kMaxScratchDevices);
  ScratchSlot& slot = g_scratch[dev];
  std::lock_guard<std::mutex> lock(slot.mu);
  if (slot.ptr == nullptr) {
    void* p = nullptr;
    hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err == hipSuccess) {
      hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, s, static_cast<uint32_t*>(p), kScratchKeys);
      err = hipGetLastError();
    }
    if (err != hipSuccess) {
      set_error("nkv_decode_step_noalloc: scratch set-up failed: %s", hipGetErrorString(err));
      return NKV_ERR_HIP;
    }
    slot.ptr = p;
  }
  *out = static_cast<char*>(slot.ptr);
  return NKV_OK;
}

// After a failed launch part-way through a range (NKV_ERR_HIP: the
// arguments were checked and a scorer may have run), the range's score keys
// may hold the scorer's maxima: clear them on the range's stream, so the
// workspace is zero for the next call as the entry points promise.  An
// argument error returns before anything is enqueued and clears nothing.
int clear_keys_after_failure(int rc, uint32_t* keys, int64_t n, hipStream_t s) {
  if (rc == NKV_ERR_HIP) {
    hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, s, keys, n);
    (void)hipGetLastError();
  }
  return rc;
}

// Events of this host thread for the current device, created on first use
// (disable-timing events; they live as long as the thread).
int step_events(int n, hipEvent_t* out) {
  struct PerDevice {
    int dev;
    std::vector<hipEvent_t> ev;
  };
  static thread_local std::vector<PerDevice> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  PerDevice* pd = nullptr;
  for (auto& c : cache)
    if (c.dev == dev) pd = &c;
  if (pd == nullptr) {
    cache.push_back(PerDevice{dev, {}});
    pd = &cache.back();
  }
  while (static_cast<int>(pd->ev.size()) < n) {
    hipEvent_t e;
    // the joins are between streams of one device: no system-scope fence
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventDisableSystemFence) != hipSuccess)
      return -1;
    pd->ev.push_back(e);
  }
  for (int i = 0; i < n; ++i) out[i] = pd->ev[i];
  return 0;
}

int hip_fail(hipError_t e, const char* what) {
  set_error("%s: %s", what, hipGetErrorString(e));
  return NKV_ERR_HIP;
}

}  // namespace
}  // namespace nkv

using namespace nkv;

extern "C" int64_t nkv_decode_step_workspace_floats(int num_layers, int num_kv_heads, int num_heads,
                                                    int splits, int nstreams) {
  if (nstreams < 1 || nstreams > kMaxStepStreams || num_layers < 1) return 0;
  const int per = (num_layers + nstreams - 1) / nstreams;  // the largest range
  const int64_t f = nkv_attend_workspace_floats(per, num_kv_heads, num_heads, 1, splits);
  return f > 0 ? f * nstreams : 0;
}

extern "C" int nkv_decode_step(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                               const uint16_t* k_new, const uint16_t* v_new, int nblocks,
                               const int32_t* protected_ids, int n_protected, int k, int n_hist,
                               int sink_len, int write_slot, int ring_base, int rec_lo, int rec_len,
                               float scale, int splits, uint32_t* score_keys, int32_t* out_ids,
                               float* partial_ws, uint16_t* out, int nstreams, void* const* streams) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_ARG(nstreams >= 1 && nstreams <= kMaxStepStreams, "nkv_decode_step: nstreams must be in [1, %d] (got %d)",
                kMaxStepStreams, nstreams);
  NKV_CHECK_ARG(streams != nullptr, "nkv_decode_step: streams is NULL");
  NKV_CHECK_ARG(q != nullptr && k_new != nullptr && v_new != nullptr && score_keys != nullptr &&
                    out_ids != nullptr && out != nullptr,
                "nkv_decode_step: q, k_new, v_new, score_keys, out_ids and out must be non-NULL");
  NKV_CHECK_ARG(n_hist >= 1 && n_hist <= k, "nkv_decode_step: n_hist must be in [1, k] (got %d, k=%d)", n_hist, k);
  NKV_CHECK_ARG(splits != 1 ? partial_ws != nullptr : true, "nkv_decode_step: splits != 1 needs partial_ws");
  const int nranges = nstreams < num_layers ? nstreams : num_layers;

  // contiguous per-layer strides: q/out [L][1][Hq][D], k/v [L][1][Hkv][D],
  // ids [L][k], keys [L][nblocks]
  const int64_t q_ls = static_cast<int64_t>(st->num_heads) * kHeadDim;
  const int64_t kv_ls = static_cast<int64_t>(st->num_kv_heads) * kHeadDim;
  const int per = (num_layers + nranges - 1) / nranges;
  const int64_t ws_range = nkv_attend_workspace_floats(per, st->num_kv_heads, st->num_heads, 1, splits);

  // the attention arguments are checked before anything is enqueued (the
  // selection's step form leaves the keys for the attention launch to clear)
  for (int r = 0; r < nranges; ++r) {
    const int l0 = static_cast<int>(static_cast<int64_t>(r) * num_layers / nranges);
    const int l1 = static_cast<int>(static_cast<int64_t>(r + 1) * num_layers / nranges);
    attend_detail::AttendParams p;
    rc = fill_attend_params("nkv_decode_step", st, layer0 + l0, l1 - l0, q + l0 * q_ls, q_ls, 1, k_new + l0 * kv_ls,
                            v_new + l0 * kv_ls, kv_ls, 1, write_slot, out_ids + static_cast<int64_t>(l0) * k, k,
                            n_hist, nullptr, 0, sink_len, ring_base, rec_lo, rec_len, scale, splits,
                            partial_ws ? partial_ws + r * ws_range : nullptr, out + l0 * q_ls, &p);
    if (rc != NKV_OK) return rc;
  }

  hipStream_t s0 = reinterpret_cast<hipStream_t>(streams[0]);
  hipEvent_t ev[kMaxStepStreams];
  if (nranges > 1) {
    NKV_CHECK_ARG(step_events(nranges, ev) == 0, "nkv_decode_step: could not create stream events");
    const hipError_t e = hipEventRecord(ev[0], s0);
    if (e != hipSuccess) return hip_fail(e, "nkv_decode_step: hipEventRecord");
  }
  for (int r = 0; r < nranges; ++r) {
    const int l0 = static_cast<int>(static_cast<int64_t>(r) * num_layers / nranges);
    const int l1 = static_cast<int>(static_cast<int64_t>(r + 1) * num_layers / nranges);
    const int nl = l1 - l0;
    void* sr = streams[r];
    if (r > 0) {
      const hipError_t e = hipStreamWaitEvent(reinterpret_cast<hipStream_t>(sr), ev[0], 0);
      if (e != hipSuccess) return hip_fail(e, "nkv_decode_step: hipStreamWaitEvent");
    }
    // the selection's step form leaves the keys for the attention launch to clear
    uint32_t* keys = score_keys + static_cast<int64_t>(l0) * nblocks;
    const int64_t nkeys = static_cast<int64_t>(nl) * nblocks;
    rc = select_impl(st, layer0 + l0, nl, q + l0 * q_ls, q_ls, 1, 0, nblocks, protected_ids, n_protected, k,
                     NKV_ORDER_SCORE_DESC, keys, nullptr, out_ids + static_cast<int64_t>(l0) * k, nullptr, true, sr);
    if (rc != NKV_OK) return clear_keys_after_failure(rc, keys, nkeys, reinterpret_cast<hipStream_t>(sr));
    const bool step_keys = select_step_form(1, n_protected, nblocks);
    rc = attend_impl(st, layer0 + l0, nl, q + l0 * q_ls, q_ls, 1, k_new + l0 * kv_ls, v_new + l0 * kv_ls, kv_ls,
                     1, write_slot, out_ids + static_cast<int64_t>(l0) * k, k, n_hist, nullptr, 0, sink_len,
                     ring_base, rec_lo, rec_len, scale, splits, partial_ws ? partial_ws + r * ws_range : nullptr,
                     out + l0 * q_ls, step_keys ? keys : nullptr, nblocks, sr);
    if (rc != NKV_OK) return clear_keys_after_failure(rc, keys, nkeys, reinterpret_cast<hipStream_t>(sr));
    if (r > 0) {
      const hipError_t e = hipEventRecord(ev[r], reinterpret_cast<hipStream_t>(sr));
      if (e != hipSuccess) return hip_fail(e, "nkv_decode_step: hipEventRecord");
    }
  }
  for (int r = 1; r < nranges; ++r) {
    const hipError_t e = hipStreamWaitEvent(s0, ev[r], 0);
    if (e != hipSuccess) return hip_fail(e, "nkv_decode_step: hipStreamWaitEvent");
  }
  return NKV_OK;
}

extern "C" int nkv_decode_step_noalloc(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                                       const uint16_t* k_new, const uint16_t* v_new, int nblocks,
                                       const int32_t* protected_ids, int n_protected, int k, int n_hist,
                                       int sink_len, int write_slot, int ring_base, int rec_lo, int rec_len,
                                       float scale, int splits, int32_t* out_ids, uint16_t* out, void* stream) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_ARG(nblocks >= 1, "nkv_decode_step_noalloc: nblocks must be >= 1 (got %d)", nblocks);
  NKV_CHECK_ARG(splits >= 0 && splits <= 64, "nkv_decode_step_noalloc: splits must be in [0, 64] (got %d; 0 = stream form)", splits);
  NKV_CHECK_ARG(static_cast<int64_t>(num_layers) * nblocks <= kScratchKeys,
                "nkv_decode_step_noalloc: num_layers x nblocks = %lld exceeds the scratch's %lld score keys",
                static_cast<long long>(num_layers) * nblocks, static_cast<long long>(kScratchKeys));
  const int64_t part = nkv_attend_workspace_floats(num_layers, st->num_kv_heads, st->num_heads, 1, splits);
  NKV_CHECK_ARG(part <= kScratchPartialFloats,
                "nkv_decode_step_noalloc: the split partials need %lld floats, the scratch holds %lld "
                "(fewer layers or splits)",
                static_cast<long long>(part), static_cast<long long>(kScratchPartialFloats));
  NKV_CHECK_ARG(q != nullptr && k_new != nullptr && v_new != nullptr && out_ids != nullptr && out != nullptr,
                "nkv_decode_step_noalloc: q, k_new, v_new, out_ids and out must be non-NULL");
  NKV_CHECK_ARG(n_hist >= 1 && n_hist <= k, "nkv_decode_step_noalloc: n_hist must be in [1, k] (got %d, k=%d)",
                n_hist, k);
  char* base = nullptr;
  rc = scratch_address(reinterpret_cast<hipStream_t>(stream), &base);
  if (rc != NKV_OK) return rc;
  void* streams[1] = {stream};
  return nkv_decode_step(st, layer0, num_layers, q, k_new, v_new, nblocks, protected_ids, n_protected, k, n_hist,
                         sink_len, write_slot, ring_base, rec_lo, rec_len, scale, splits,
                         reinterpret_cast<uint32_t*>(base), out_ids, reinterpret_cast<float*>(base + kScratchKeyBytes),
                         out, 1, streams);
}
