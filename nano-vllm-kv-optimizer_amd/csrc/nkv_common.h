// Shared helpers for the NanoKV gfx950 kernels: bf16 conversions, the
// per-thread error message, and argument-check macros used by every entry
// point of include/nanokv.h.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/nanokv.h"

namespace nkv {

constexpr int kHeadDim = 128;   // D: fixed by the MFMA / lane tilings
constexpr int kBlock = 64;      // B: tokens per history block
constexpr int kWave = 64;       // CDNA wavefront width

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);

#define NKV_CHECK_ARG(cond, ...)                  \
  do {                                            \
    if (!(cond)) {                                \
      ::nkv::set_error(__VA_ARGS__);              \
      return NKV_ERR_ARG;                         \
    }                                             \
  } while (0)

#define NKV_CHECK_SUPPORTED(cond, ...)            \
  do {                                            \
    if (!(cond)) {                                \
      ::nkv::set_error(__VA_ARGS__);              \
      return NKV_ERR_UNSUPPORTED;                 \
    }                                             \
  } while (0)

// Launch-status check after a kernel enqueue.
int launch_status(const char* what);

// Validate the fields of a store descriptor that every entry point relies on.
int check_store(const nkv_store* st, int layer0, int num_layers);

// Compute units of the current device (cached per thread); 0 on error.
int device_cus();

// nkv_select with the decode step's option: with step set (and one query, no
// raw scores or values, at most 64 protected ids, at most 2048 blocks) the
// scorer leaves the protected blocks' keys at zero and the top-k neither
// reads the protected list nor clears the keys -- the caller's attention
// launch must clear them (AttendParams.zero_keys).  Same ids either way.
// With uo non-NULL (per_query, nq <= 16, k <= 64, nblocks <= 2048) the per-query
// top-k and the union of the selections (nkv_select_union's outputs) are one
// launch.
struct UnionOut {
  int umax;
  int32_t* out_union;
  int32_t* out_count;
  uint8_t* out_allowed;
};
int select_impl(const nkv_store* st, int layer0, int num_layers, const uint16_t* q, int64_t q_layer_stride, int nq,
                int per_query, int nblocks, const int32_t* protected_ids, int n_protected, int k, int order,
                uint32_t* score_keys, float* out_scores, int32_t* out_ids, float* out_vals, bool step,
                void* stream, const UnionOut* uo = nullptr);
// Whether select_impl takes the step form for these sizes (out_scores and
// out_vals NULL, per_query 0).
bool select_step_form(int nq, int n_protected, int nblocks);

// nkv_attend; with zero_keys non-NULL the launch also clears
// zero_keys[l][0 .. zero_n) of every layer l it attends.
int attend_impl(const nkv_store* st, int layer0, int num_layers, const uint16_t* q, int64_t q_layer_stride, int tq,
                const uint16_t* k_new, const uint16_t* v_new, int64_t kv_layer_stride, int n_chunk, int write_slot,
                const int32_t* ids, int64_t ids_layer_stride, int n_hist, const uint8_t* allowed,
                int64_t allowed_layer_stride, int sink_len, int ring_base, int rec_lo, int rec_len, float scale,
                int splits, float* partial_ws, uint16_t* out, uint32_t* zero_keys, int zero_n, void* stream);

// ------------------------------------------------------------ bf16 / fp16 --
__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// fp32 -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Monotone uint32 key of an fp32 score: larger score -> larger key.
// -0.0 is folded onto +0.0; every NaN maps to the canonical quiet NaN, which
// sorts above +inf (torch.topk's NaN convention).
__device__ __forceinline__ uint32_t score_key(float s) {
  s = s + 0.0f;
  uint32_t u = __float_as_uint(s);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_score(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

}  // namespace nkv
