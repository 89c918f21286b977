// Error state and descriptor checks shared by all NanoKV entry points.
#include "nkv_common.h"

namespace nkv {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return NKV_ERR_HIP;
  }
  return NKV_OK;
}

int check_store(const nkv_store* st, int layer0, int num_layers) {
  NKV_CHECK_ARG(st != nullptr, "store descriptor is NULL");
  NKV_CHECK_SUPPORTED(st->head_dim == kHeadDim, "head_dim must be %d (got %d)", kHeadDim, st->head_dim);
  NKV_CHECK_SUPPORTED(st->block_size == kBlock, "block_size must be %d (got %d)", kBlock, st->block_size);
  NKV_CHECK_ARG(st->num_kv_heads >= 1 && st->num_heads >= st->num_kv_heads &&
                    st->num_heads % st->num_kv_heads == 0,
                "num_heads (%d) must be a positive multiple of num_kv_heads (%d)",
                st->num_heads, st->num_kv_heads);
  const int g = st->num_heads / st->num_kv_heads;
  NKV_CHECK_SUPPORTED(g == 1 || g == 2 || g == 4 || g == 8 || g == 16,
                      "GQA group size %d not in {1,2,4,8,16}", g);
  NKV_CHECK_SUPPORTED(st->r == 1 || st->r == 2 || st->r == 4 || st->r == 8,
                      "r must be 1, 2, 4 or 8 (got %d)", st->r);
  NKV_CHECK_ARG(st->cap_blocks >= 1, "cap_blocks must be >= 1");
  NKV_CHECK_ARG(st->sink_tokens >= 0 && st->recent_tokens >= 1,
                "sink_tokens must be >= 0 and recent_tokens >= 1");
  NKV_CHECK_ARG(st->kv_format >= NKV_KV_BF16 && st->kv_format <= NKV_KV_INT8_TOKEN,
                "unknown kv_format %d", st->kv_format);
  NKV_CHECK_ARG(num_layers >= 1 && layer0 >= 0 && layer0 + num_layers <= st->num_layers,
                "layer range [%d, %d) outside [0, %d)", layer0, layer0 + num_layers, st->num_layers);
  NKV_CHECK_ARG(st->hist_k && st->hist_v && st->reps && st->recent_k && st->recent_v,
                "store has a NULL history / reps / recent pointer");
  NKV_CHECK_ARG(st->sink_tokens == 0 || (st->sink_k && st->sink_v), "store has a NULL sink pointer");
  if (st->kv_format == NKV_KV_INT8_CHANNEL)
    NKV_CHECK_ARG(st->k_scale && st->v_scale, "int8 channel format needs k_scale and v_scale");
  if (st->kv_format == NKV_KV_INT8_TOKEN)
    NKV_CHECK_ARG(st->k_tscale && st->v_tscale, "int8 token format needs k_tscale and v_tscale");
  return NKV_OK;
}

int device_cus() {
  static thread_local int dev_cached = -1, cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev != dev_cached) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus = n;
    dev_cached = dev;
  }
  return cus;
}

}  // namespace nkv

extern "C" int nkv_abi_version(void) { return NKV_ABI_VERSION; }

extern "C" int nkv_host_device_pointer(const void* host_ptr, void** device_ptr) {
  NKV_CHECK_ARG(host_ptr != nullptr && device_ptr != nullptr,
                "nkv_host_device_pointer: host_ptr and device_ptr must be non-NULL");
  *device_ptr = nullptr;
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, host_ptr);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // an unknown (pageable) pointer is an argument error, not a fault
    ::nkv::set_error("nkv_host_device_pointer: %p is not memory of the HIP runtime (%s)", host_ptr,
                     hipGetErrorString(e));
    return NKV_ERR_ARG;
  }
  NKV_CHECK_ARG(attr.type == hipMemoryTypeHost,
                "nkv_host_device_pointer: %p is not pinned host memory (memory type %d)", host_ptr,
                static_cast<int>(attr.type));
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, const_cast<void*>(host_ptr), 0);
  if (e != hipSuccess || d == nullptr) {
    (void)hipGetLastError();
    ::nkv::set_error("nkv_host_device_pointer: %p is not mapped for the device (%s)", host_ptr,
                     hipGetErrorString(e));
    return NKV_ERR_ARG;
  }
  *device_ptr = d;
  return NKV_OK;
}
extern "C" const char* nkv_last_error(void) { return nkv::g_last_error; }
