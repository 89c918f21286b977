// Segment machinery shared by the few-query attention kernel (nkv_attend.hip)
// and the many-query prefill kernel (nkv_prefill.hip): the launch parameters
// and the description of one attended segment (history block, sink piece,
// physical ring piece or chunk piece).
#pragma once

#include "nkv_common.h"

namespace nkv {
namespace attend_detail {

#ifndef NKV_ATTEND_DECODE_WAVES
#define NKV_ATTEND_DECODE_WAVES 2  // waves per SIMD the 4-row (decode) variants are built for (3 spills and measured slower)
#endif
constexpr int kAttendWaves = 4;
constexpr int kAttendThreads = kAttendWaves * kWave;
constexpr int kPRow = 20;        // floats per key row of the p tile in LDS (16 rows + pad)
constexpr int kPartStride = 130; // floats per partial row: m, l, acc[128]
constexpr int kMaxRows = 16;     // MFMA N: query rows per group
constexpr int kWideRows = 32;    // query rows per group of the two-tile (wide) few-query kernel
constexpr int kStreamRows = 4;   // rows per partial record of the 4-row kernel's stream form
constexpr int64_t kStreamWavesMax = 2048;  // wavefronts a stream-form launch uses at most
constexpr int kWidePlanSlotsMax = 512;     // resident wide-kernel workgroups a tiered plan fills at most

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum SegType { kSegHist = 0, kSegSink = 1, kSegRecent = 2, kSegChunk = 3 };

struct AttendParams {
  const void* hist_k;
  const void* hist_v;
  int64_t hist_ls;
  const uint16_t* sink_k;
  const uint16_t* sink_v;
  int64_t sink_ls;
  uint16_t* rec_k;
  uint16_t* rec_v;
  int64_t rec_ls;
  const float* k_scale;     // [L][Hkv][D]
  const float* v_scale;     // [L][Hkv][cap]
  const uint16_t* k_tscale; // [L][Hkv][cap*64]
  const uint16_t* v_tscale;
  const uint16_t* q;
  int64_t q_ls;
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t kv_ls;
  const int32_t* ids;
  int64_t ids_ls;
  const uint8_t* allowed;   // [tq][n_hist] per layer, layer stride allowed_ls (0: shared)
  int64_t allowed_ls;
  float* partial;
  uint16_t* out;
  int hkv, G, cap, S, R;
  int tq, qpg, nqg;
  int n_chunk, write_slot;
  int n_hist, sink_len, ring_base, rec_lo, rec_len;
  // non-null: per-layer ring starts in device memory, used instead of
  // write_slot / ring_base (write slot = start, ring base = start + 1 mod R)
  const int32_t* ring_start;
  int n_sink_seg, n_rec_seg, nseg;
  int splits;
  float scale_log2;
  // chunk visibility: query t sees chunk token c iff c - causal_off <= t
  // (0 for prefill / verify / decode chunks; caller-packed keys put their
  // causal start here) and, with tok_mask != NULL, tok_mask[t][c] == 0
  // (uint8 [tq][n_chunk], nonzero = hidden)
  int causal_off;
  const uint8_t* tok_mask;
  // non-null: the layer's first workgroup clears zero_keys[layer][0 .. zero_n)
  // (the decode step's score keys, consumed by the top-k launch before it)
  uint32_t* zero_keys;
  int zero_n;
  // per-query-tile selection (matrix-core kernel): with sel_tile > 0 the
  // queries t of tile t / sel_tile attend the history blocks
  // ids[layer][tile * ids_tile_ls + i]
  int64_t ids_tile_ls;
  int sel_tile;
  // few-query kernels: partial records per (group, split) -- the group's row
  // capacity (kMaxRows, or kWideRows for the wide kernel; 4 in the stream
  // form)
  int prow;
  // the 4-row kernel's stream form (stream_wpg > 0): stream_wpg wavefronts
  // per (layer, KV head, query group); wavefront j of group g attends its
  // segments [j nseg / wpg, (j + 1) nseg / wpg) and writes record g wpg + j
  int stream_wpg;
  int nlayers;
  // the wide kernel's tiered split plan (wide_sa > 0): groups [0, wide_ga)
  // take wide_sa splits each (records g wide_sa + s), the rest wide_sb
  // (records after those), one workgroup per (group, split) in that order
  int wide_ga, wide_sa, wide_sb;
};

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

// K/V loads.  NT: non-temporal (a decode step reads each selected block once,
// so the stream should not evict the lines that are reused: the next step's
// representatives, queries, ids, partials).
template <bool NT>
__device__ __forceinline__ uint4 kv_load16(const char* p) {
  if (NT) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  return *reinterpret_cast<const uint4*>(p);
}
template <bool NT>
__device__ __forceinline__ uint2 kv_load8(const char* p) {
  if (NT) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    return make_uint2(v.x, v.y);
  }
  return *reinterpret_cast<const uint2*>(p);
}

// Max / sum of x over the four 16-lane rows of the wavefront (lanes l, l ^ 16,
// l ^ 32, l ^ 48), the result in every lane.  gfx950's row swaps
// (v_permlane16_swap / v_permlane32_swap: with both operands x, the pair holds
// x of lane l & ~16 and of lane l | 16, resp. & ~32 and | 32) stay in the VALU,
// where a shuffle through ds_bpermute waits on the LDS pipeline.
__device__ __forceinline__ float max_over_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 8 signed bytes -> 8 bf16 (exact: |x| <= 128 has <= 8 significant bits).
// One byte-select conversion per value and one bf16 pack per pair
// (v_cvt_f32_i32 with a sign-extended byte operand, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint4 i8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t src = ((i < 2) ? lo : hi) >> ((i & 1) * 16);
    const float f0 = static_cast<float>(static_cast<int8_t>(src & 0xffu));
    const float f1 = static_cast<float>(static_cast<int8_t>((src >> 8) & 0xffu));
    const bf16x2_t v = {static_cast<__bf16>(f0), static_cast<__bf16>(f1)};
    o[i] = __builtin_bit_cast(uint32_t, v);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// A segment: `len` rows starting at kbase / vbase, row stride `rowb` bytes;
// rows >= len are never loaded (indices are clamped).  `vlen` = rows that may
// be valid (a history block with an out-of-range id has vlen 0).
struct Seg {
  int type;
  int len;
  int vlen;
  int off;   // sink / chunk: first token; recent: first physical slot
  int blk;   // history block id
  int u;     // history segment index (column of `allowed`)
  int rowb;
  const char* kbase;
  const char* vbase;
};

// Segment s of (layer, KV head h); for a history segment `blk` is its block
// id (ids[layer][s]).
template <int FMT>
__device__ __forceinline__ Seg make_seg_blk(const AttendParams& p, int layer, int h, int s, int blk) {
  Seg g;
  g.blk = 0;
  g.u = 0;
  g.off = 0;
  if (s < p.n_hist) {
    constexpr int64_t elem = (FMT == NKV_KV_BF16) ? 2 : 1;
    g.type = kSegHist;
    g.len = kBlock;
    g.vlen = kBlock;
    g.u = s;
    if (blk < 0 || blk >= p.cap) {  // never read outside the history
      blk = 0;
      g.vlen = 0;
    }
    g.blk = blk;
    const int64_t off = (p.hist_ls * layer + (static_cast<int64_t>(h) * p.cap + blk) * kBlock * kHeadDim) * elem;
    g.kbase = static_cast<const char*>(p.hist_k) + off;
    g.vbase = static_cast<const char*>(p.hist_v) + off;
    g.rowb = kHeadDim * static_cast<int>(elem);
    return g;
  }
  s -= p.n_hist;
  g.rowb = kHeadDim * 2;
  if (s < p.n_sink_seg) {
    g.type = kSegSink;
    g.off = s * kBlock;
    g.len = min(kBlock, p.sink_len - g.off);
    g.vlen = g.len;
    const int64_t off = p.sink_ls * layer + (static_cast<int64_t>(h) * p.S + g.off) * kHeadDim;
    g.kbase = reinterpret_cast<const char*>(p.sink_k + off);
    g.vbase = reinterpret_cast<const char*>(p.sink_v + off);
    return g;
  }
  s -= p.n_sink_seg;
  if (s < p.n_rec_seg) {
    g.type = kSegRecent;
    g.off = s * kBlock;
    g.len = min(kBlock, p.R - g.off);
    g.vlen = g.len;
    const int64_t off = p.rec_ls * layer + (static_cast<int64_t>(h) * p.R + g.off) * kHeadDim;
    g.kbase = reinterpret_cast<const char*>(p.rec_k + off);
    g.vbase = reinterpret_cast<const char*>(p.rec_v + off);
    return g;
  }
  s -= p.n_rec_seg;
  g.type = kSegChunk;
  g.off = s * kBlock;
  g.len = min(kBlock, p.n_chunk - g.off);
  g.vlen = g.len;
  g.rowb = p.hkv * kHeadDim * 2;
  const int64_t off = p.kv_ls * layer + (static_cast<int64_t>(g.off) * p.hkv + h) * kHeadDim;
  g.kbase = reinterpret_cast<const char*>(p.k_new + off);
  g.vbase = reinterpret_cast<const char*>(p.v_new + off);
  return g;
}

template <int FMT>
__device__ __forceinline__ Seg make_seg(const AttendParams& p, int layer, int h, int s) {
  const int blk = s < p.n_hist ? p.ids[static_cast<int64_t>(layer) * p.ids_ls + s] : 0;
  return make_seg_blk<FMT>(p, layer, h, s, blk);
}

}  // namespace attend_detail

// Launch the few-query kernel (+ split merge) / the matrix-core kernel (+
// split merge) over filled parameters; hkv / kv_format describe the keys.
int launch_grouped(int hkv, int kv_format, int num_layers, int tq, attend_detail::AttendParams& p,
                   hipStream_t s);
int launch_prefill(int hkv, int kv_format, int num_layers, int tq, attend_detail::AttendParams& p,
                   hipStream_t s);

// Validates the arguments shared by nkv_attend and nkv_prefill_attend and
// fills the launch parameters (everything except the query grouping, which
// each kernel chooses).  Returns NKV_OK or an error code with the message set.
int fill_attend_params(const char* who, const nkv_store* st, int layer0, int num_layers,
                       const uint16_t* q, int64_t q_layer_stride, int tq, const uint16_t* k_new,
                       const uint16_t* v_new, int64_t kv_layer_stride, int n_chunk, int write_slot,
                       const int32_t* ids, int64_t ids_layer_stride, int n_hist,
                       const uint8_t* allowed, int64_t allowed_layer_stride, int sink_len,
                       int ring_base, int rec_lo, int rec_len,
                       float scale, int splits, float* partial_ws, uint16_t* out,
                       attend_detail::AttendParams* p);

}  // namespace nkv
