// Staging of attention segments through LDS on gfx950, used by the
// many-query kernel (nkv_prefill.hip) and the few-query kernel's matrix-core
// P.V (nkv_attend.hip): the stage-buffer layout, direct global -> LDS copies
// of a bf16 segment, bf16 packing and branch-free visibility bounds.
#pragma once

#include "nkv_attend_common.h"

namespace nkv {
namespace stage {
using namespace attend_detail;

constexpr int kTileBytes = kBlock * kHeadDim * 2;
constexpr int kBufBytes = 2 * kTileBytes;        // K tile + V tile
constexpr int kRsrcWord3 = 0x00020000;           // raw buffer, 32-bit data format

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// LDS layout of one stage buffer (bytes), both tiles key-major, 256 B a row:
//   K tile [0, 16384): key r at r * 256, its 16-byte chunk c (dims 8c .. 8c+7)
//          at chunk position c ^ (r & 15);
//   V tile [16384, 32768): key k at 16384 + k * 256, chunk c at position
//          c ^ (2 (k & 3)).
// The swizzles make the 16-byte K reads (8 lanes, 8 keys) and the 8-byte
// transposing V reads (16 lanes, 4 keys x 16 dims) free of bank conflicts.

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// Bounds-checked descriptor of rows [0, len) of a segment: reads past the
// last row return zero, and every read of a row stays inside it.  With
// live == false the range is empty: the copy still issues its instructions
// but reads nothing (zeros land in LDS).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t seg_rsrc(const char* base, const Seg& g, bool live = true) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, live ? g.len * g.rowb : 0, kRsrcWord3);
}

// bf16 segment -> LDS buffer `buf` without registers.  Wavefront w copies K
// and V rows 16w .. 16w+15, four rows (1 KiB) per instruction; lane u lands
// at buf + 16 u, so it fetches the global chunk that the swizzle puts there.
//   kx[i] = byte offset of that chunk in K row 16w + 4i + (u >> 4); vx likewise for V.
__device__ __forceinline__ void dma_segment(const Seg& g, char* buf, int wave, int lane, const int (&kx)[4],
                                            int vx, bool live = true) {
  const __amdgpu_buffer_rsrc_t rk = seg_rsrc(g.kbase, g, live);
  const __amdgpu_buffer_rsrc_t rv = seg_rsrc(g.vbase, g, live);
  const int rowo = (16 * wave + (lane >> 4)) * g.rowb;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    char* dst = buf + (16 * wave + 4 * i) * 256;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)dst, 16, rowo + kx[i], 4 * i * g.rowb, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(dst + kTileBytes), 16, rowo + vx, 4 * i * g.rowb, 0, 0);
  }
}

// Raw buffer descriptor words of bytes [base, base + bytes): reads at or past
// `bytes` return zero.
// The words are read from the first active lane: they are uniform by
// construction, and the copy's descriptor operand must sit in SGPRs.
typedef uint32_t rsrc_words __attribute__((ext_vector_type(4)));
__device__ __forceinline__ rsrc_words rsrc_of(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  auto uni = [](uint32_t x) { return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x))); };
  return rsrc_words{uni(static_cast<uint32_t>(a)), uni(static_cast<uint32_t>(a >> 32) & 0xffffu), uni(bytes),
                    static_cast<uint32_t>(kRsrcWord3)};
}

// One global -> LDS copy, 16 bytes a lane (buffer_load_dwordx4 ... lds): lane
// u's bytes at `voffset` of the buffer land at LDS address lds + 16 u.  Issued
// as inline assembly, so that the compiler (which counts such copies against
// all of LDS) adds no waits of its own: the kernels order them with explicit
// vmcnt waits.  The memory clobber keeps every LDS access on its side of the
// copy.  M0 (the LDS base, read when the copy issues) is restored after it;
// the s_nops cover the descriptor-write and M0-write hazards.
__device__ __forceinline__ void lds_copy16(rsrc_words rsrc, const char* lds, int voffset) {
  const uint32_t m0 = static_cast<uint32_t>(
      __builtin_amdgcn_readfirstlane(static_cast<int>(reinterpret_cast<uintptr_t>((lds_void*)lds))));
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_nop 4\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m0), "v"(voffset), "s"(rsrc)
      : "memory");
}
// The same, 4 bytes a lane (buffer_load_dword ... lds): lane u lands at lds + 4 u.
__device__ __forceinline__ void lds_copy4(rsrc_words rsrc, const char* lds, int voffset) {
  const uint32_t m0 = static_cast<uint32_t>(
      __builtin_amdgcn_readfirstlane(static_cast<int>(reinterpret_cast<uintptr_t>((lds_void*)lds))));
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_nop 4\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m0), "v"(voffset), "s"(rsrc)
      : "memory");
}

// +inf when d <= 0 (key visible), -inf when d > 0: min(S, bound) masks S
// without lane masks (no SGPR pairs).
__device__ __forceinline__ float vis_bound(int d) {
  return __int_as_float(0x7F800000 | ((0 - d) & static_cast<int>(0x80000000u)));
}

}  // namespace stage
}  // namespace nkv
