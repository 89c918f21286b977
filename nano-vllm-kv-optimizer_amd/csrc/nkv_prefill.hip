// Segmented causal GQA attention for many queries: the attention of a
// chunked-prefill step (and of long verify chunks), on the matrix cores.
//
// Keys are the same segments as the few-query kernel (nkv_attend.hip): the
// selected history blocks read in place (bf16, or int8 dequantised to bf16
// exactly as the reference packs them), the sink, the recent ring in physical
// 64-slot pieces masked to the logical window, and the chunk itself, causal
// (query t sees chunk token c iff c <= t).  The chunk segments a workgroup
// visits stop at its last query token.
//
// Work split: one workgroup (4 wavefronts) per (layer, KV head, query tile).
// A query tile is 128 columns = 128/G tokens x the G query heads of the KV
// head, so every K/V tile staged in LDS serves all G heads.  Wavefront w owns
// columns 32w..32w+31 (two 16-column MFMA tiles).  Workgroups are ordered so
// that the linear id cycles over the KV heads (one head per XCD when
// Hkv = 8, keeping that head's keys in one L2) and the longest causal tiles
// start first.
//
// Per 64-key segment (double-buffered LDS, one barrier per segment):
//   * staging: rows go global -> LDS directly (buffer_load ... lds, no
//     registers; bounds-checked descriptors read rows past the segment as
//     zero, so no index is clamped).  int8 history rows land raw with their
//     scales and are dequantised to bf16 in LDS after the copy.  The next
//     segment is in flight while the current one is computed;
//   * S^T = K . Q^T: v_mfma_f32_16x16x32_bf16, A = 16 keys x 32 dims read from
//     the K tile, B = 32 dims x 16 columns held in registers all along;
//   * online softmax in fp32 per column (exp2, scale folded in); each lane's
//     column is fixed, so the running max and the rescale stay in the lane;
//   * O^T += V^T . P^T: A = 16 dims x 32 keys assembled from the key-major V
//     tile with two transposing LDS reads (ds_read_b64_tr_b16), B = the
//     lane's own probabilities rounded to bf16 (the 32-key contraction index
//     is ordered as the S^T accumulator holds the keys, so P never leaves the
//     registers).
//
// The reference runs this as flash-attention over the packed
// [selected | sink | recent | chunk] keys with bottom-right causal masking
// (nanovllm/sparse/m12_runtime.py:592-651, :809-839); the fp32 masked path
// (:875-896) is the same function.
#include <type_traits>

#include "nkv_stage.h"

namespace nkv {
namespace {
using namespace attend_detail;
using namespace stage;

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;     // 256
constexpr int kPfCols = 128;                     // (token, head) columns per workgroup
// split partial record of one column: m (reference max, log2 units), l, two
// pad words, acc[128] (16-byte aligned for vector stores)
constexpr int kPfPart = 4 + kHeadDim;

// 8 int8 codes (lo, hi) -> 8 x bf16(code * scale[e]), rounded to nearest even.
__device__ __forceinline__ u32x4 dequant8(uint32_t lo, uint32_t hi, const float (&sc)[8]) {
  float f[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t w = e < 4 ? lo : hi;
    f[e] = static_cast<float>(static_cast<int8_t>((w >> ((e & 3) * 8)) & 0xffu)) * sc[e];
  }
  return u32x4{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]), pack_bf16(f[6], f[7])};
}

// int8 history block: the raw codes (and the scales) are copied into the
// destination buffer first, then dequantised in place by dequant_i8 once the
// copies have landed.  Staging layout inside the buffer:
//   [0, 512)        K scales (per-token fp16 x 64, or per-channel fp32 x 128)
//   [512, 768)      V per-token fp16 scales x 64
//   [16384, 24576)  raw K codes, 64 rows x 128 B
//   [24576, 32768)  raw V codes, 64 rows x 128 B
constexpr int kI8Scales = 0;
constexpr int kI8VScales = 512;
constexpr int kI8RawK = kTileBytes;
constexpr int kI8RawV = kTileBytes + kBlock * kHeadDim;

template <int FMT>
__device__ __forceinline__ void dma_i8_segment(const AttendParams& p, const Seg& g, int lh, char* buf, int wave,
                                               int lane) {
  const __amdgpu_buffer_rsrc_t rk = seg_rsrc(g.kbase, g);
  const __amdgpu_buffer_rsrc_t rv = seg_rsrc(g.vbase, g);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int o = (2 * wave + i) * 1024;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(buf + kI8RawK + o), 16, lane * 16, o, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(buf + kI8RawV + o), 16, lane * 16, o, 0, 0);
  }
  if (wave == 0) {
    if (FMT == NKV_KV_INT8_TOKEN) {
      // 64 fp16 scales = 128 B per tensor; lanes 32.. read past it (zeros)
      const int64_t tb = (static_cast<int64_t>(lh) * p.cap + g.blk) * kBlock;
      const __amdgpu_buffer_rsrc_t sk = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(p.k_tscale + tb), 0, kBlock * 2, kRsrcWord3);
      const __amdgpu_buffer_rsrc_t sv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(p.v_tscale + tb), 0, kBlock * 2, kRsrcWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sk, (lds_void*)(buf + kI8Scales), 4, lane * 4, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sv, (lds_void*)(buf + kI8VScales), 4, lane * 4, 0, 0, 0);
    } else {
      // 128 fp32 per-(head, dim) K scales
      const __amdgpu_buffer_rsrc_t sk = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(p.k_scale + static_cast<int64_t>(lh) * kHeadDim), 0, kHeadDim * 4, kRsrcWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sk, (lds_void*)(buf + kI8Scales), 4, lane * 4, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sk, (lds_void*)(buf + kI8Scales + 256), 4, lane * 4, 256, 0, 0);
    }
  }
}

// In-place dequantisation of a staged int8 block (the copies have landed and
// are visible): thread tid converts rows (tid >> 4) + 16 j, dims 8 c .. 8 c + 7
// (c = tid & 15) of K and V to bf16(code * scale) in the K / V tiles.
template <int FMT>
__device__ __forceinline__ void dequant_i8(const AttendParams& p, const Seg& g, int lh, char* buf, int tid) {
  const int r0 = tid >> 4;
  const int c = tid & 15;
  u32x2 kq[4], vq[4];
  float ksc[4][8], vsc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = r0 + 16 * j;
    kq[j] = *reinterpret_cast<const u32x2*>(buf + kI8RawK + r * kHeadDim + c * 8);
    vq[j] = *reinterpret_cast<const u32x2*>(buf + kI8RawV + r * kHeadDim + c * 8);
  }
  if (FMT == NKV_KV_INT8_TOKEN) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + 16 * j;
      const float ks = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(buf + kI8Scales + 2 * r));
#pragma unroll
      for (int e = 0; e < 8; ++e) ksc[j][e] = ks;
      vsc[j] = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(buf + kI8VScales + 2 * r));
    }
  } else {
    const u32x4 s0 = *reinterpret_cast<const u32x4*>(buf + kI8Scales + c * 32);
    const u32x4 s1 = *reinterpret_cast<const u32x4*>(buf + kI8Scales + c * 32 + 16);
    const float vs = p.v_scale[static_cast<int64_t>(lh) * p.cap + g.blk];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ksc[j][e] = __uint_as_float(s0[e]);
        ksc[j][e + 4] = __uint_as_float(s1[e]);
      }
      vsc[j] = vs;
    }
  }
  __syncthreads();   // every raw code and scale has been read
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = r0 + 16 * j;
    float vv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vv[e] = vsc[j];
    *reinterpret_cast<u32x4*>(buf + r * 256 + ((c ^ r0) << 4)) = dequant8(kq[j][0], kq[j][1], ksc[j]);
    *reinterpret_cast<u32x4*>(buf + kTileBytes + r * 256 + ((c ^ (2 * (r0 & 3))) << 4)) =
        dequant8(vq[j][0], vq[j][1], vv);
  }
}

// Whether any (key, column) of segment g may be invisible to the workgroup's
// tokens t0.. (otherwise the mask pass is skipped).
template <bool PACKED>
__device__ __forceinline__ bool needs_mask(const AttendParams& p, const Seg& g, int t0) {
  switch (g.type) {
    case kSegHist: return g.vlen < kBlock || p.allowed != nullptr;
    case kSegSink: return g.len < kBlock;
    case kSegRecent: return !(p.rec_len == p.R && g.len == kBlock);
    default: return PACKED ? (p.tok_mask != nullptr || g.len < kBlock || g.off + kBlock - 1 - p.causal_off > t0)
                           : (g.len < kBlock || g.off + kBlock - 1 > t0);
  }
}

// -inf for the (key, column) pairs of S that the segment hides; S[kt][ct][e]
// holds key 16 kt + 4 lg + e of column ct.  Key k of the segment is visible
// to column ct iff k <= thr[ct] (history / sink / chunk), or, for a ring
// piece, iff k < vlen and the slot's logical position lies in the window.
template <bool PACKED>
__device__ __forceinline__ void apply_mask(const AttendParams& p, const Seg& g, int lg, const int (&tcol)[2],
                                           const int (&allow)[2], f32x4 (&S)[4][2]) {
  if (g.type == kSegRecent) {
    // x = (slot - ring_base - rec_lo) mod R for slot off + key
    int a = (g.off - p.ring_base - p.rec_lo) % p.R;
    a = a < 0 ? a + p.R : a;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 16 * kt + 4 * lg + e;
        int x = a + key;
        x -= p.R & ((p.R - 1 - x) >> 31);
        const float bound = vis_bound(max(key - (g.vlen - 1), x - (p.rec_len - 1)));
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) S[kt][ct][e] = fminf(S[kt][ct][e], bound);
      }
    return;
  }
  int base[2];   // 4 lg - thr[ct]
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    int thr = g.vlen - 1;
    if (g.type == kSegChunk) thr = min(thr, tcol[ct] + (PACKED ? p.causal_off : 0) - g.off);
    else if (allow[ct] == 0) thr = -1;
    base[ct] = 4 * lg - thr;
  }
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[kt][ct][e] = fminf(S[kt][ct][e], vis_bound(base[ct] + 16 * kt + e));
  if (PACKED && g.type == kSegChunk && p.tok_mask != nullptr) {
    // caller-packed keys with a per-(query, key) mask: keys past vlen are
    // already hidden and never read; padding columns read row tq - 1
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const uint8_t* mrow = p.tok_mask + static_cast<int64_t>(min(tcol[ct], p.tq - 1)) * p.n_chunk + g.off;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = 16 * kt + 4 * lg + e;
          if (key < g.vlen && mrow[key] != 0) S[kt][ct][e] = -INFINITY;
        }
    }
  }
}

// PACKED: caller-packed keys (nkv_attend_packed): the chunk's causal start is
// causal_off and an optional per-token mask applies; its own instantiation,
// so the history paths carry none of that code.
template <int FMT, bool PACKED>
__global__ __launch_bounds__(kPfThreads, 2) void prefill_kernel(const AttendParams p, int nqt) {
  // two stage buffers as separate objects, so that the compiler can tell the
  // buffer being read from the one the asynchronous copies write
  __shared__ __attribute__((aligned(16))) char lds0[kBufBytes];
  __shared__ __attribute__((aligned(16))) char lds1[kBufBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int ln = lane & 15;   // MFMA column (query) / A-operand row
  const int lg = lane >> 4;   // MFMA k-group / accumulator row group
  const int h = blockIdx.x % p.hkv;
  const int qt = nqt - 1 - static_cast<int>(blockIdx.x) / p.hkv;
  const int layer = blockIdx.y;
  const int lh = layer * p.hkv + h;
  const int tpw = kPfCols / p.G;
  const int t0 = qt * tpw;
  const int t_last = min(t0 + tpw, p.tq) - 1;
  const int hq = p.hkv * p.G;

  // ---- loop-invariant LDS offsets (bytes) -----------------------------------
  int koff[4];   // K read (QK A operand): key 16 kt + ln, chunk 4 ks + lg; kt -> + 4096 kt
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = ln * 256 + ((((4 * ks + lg) ^ ln) & 15) << 4);
  // V transposing read (PV A operand): lane ln addresses key 4 lg + (ln >> 2)
  // (+ 32 k2 + 16 half), dims 16 dt + 4 (ln & 3) .. +4; the swizzled chunk is
  // 2 (dt ^ (ln >> 2)) + ((ln & 3) >> 1), so dt & 4 -> + 128 and dt & 3 picks vtr[]
  int vtr[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    vtr[q] = kTileBytes + (4 * lg + (ln >> 2)) * 256 + ((2 * (q ^ (ln >> 2)) + ((ln & 3) >> 1)) << 4) + 8 * (ln & 1);
  int kx[4];     // copy offsets: K row 16w + 4i + (lane >> 4), global chunk (lane & 15) ^ (row & 15)
#pragma unroll
  for (int i = 0; i < 4; ++i) kx[i] = ((ln ^ ((4 * i + lg) & 15))) << 4;
  const int vx = (ln ^ (2 * lg)) << 4;   // V row & 3 == lane >> 4

  // ---- query operands: column c = 32 wave + 16 ct + ln --------------------
  bf16x8 bq[2][4];
  int tcol[2];
  int hcol[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int c = wave * 32 + ct * 16 + ln;
    const int t = t0 + c / p.G;
    tcol[ct] = t;
    hcol[ct] = h * p.G + c % p.G;
    const uint16_t* qrow = p.q + p.q_ls * layer + (static_cast<int64_t>(t) * hq + hcol[ct]) * kHeadDim + lg * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (t < p.tq) v = *reinterpret_cast<const u32x4*>(qrow + ks * 32);
      bq[ct][ks] = __builtin_bit_cast(bf16x8, v);
    }
  }

  f32x4 acc[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc[dt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.0f, 0.0f};

  // chunk segments up to the last key visible to the tile's last token
  const int n_chunk_seg =
      p.n_chunk <= 0 ? 0
                     : (PACKED ? min((p.n_chunk + kBlock - 1) / kBlock, (t_last + p.causal_off) / kBlock + 1)
                               : t_last / kBlock + 1);
  const int nseg_all = p.n_hist + p.n_sink_seg + p.n_rec_seg + n_chunk_seg;
  // split-K: this workgroup attends segments [seg_lo, nseg) of the list
  const int split = blockIdx.z;
  const int seg_lo = static_cast<int>(static_cast<int64_t>(split) * nseg_all / p.splits);
  const int nseg = static_cast<int>(static_cast<int64_t>(split + 1) * nseg_all / p.splits);

  // staging of segment s into buffer `buf`: asynchronous copies issued by
  // begin_stage, completed (and int8 blocks dequantised) by finish_stage
  int allow_nxt[2] = {1, 1};
  auto begin_stage = [&](const Seg& g, char* buf) {
    if (FMT != NKV_KV_BF16 && g.type == kSegHist)
      dma_i8_segment<FMT>(p, g, lh, buf, wave, lane);
    else
      dma_segment(g, buf, wave, lane, kx, vx);
    if (g.type == kSegHist && p.allowed != nullptr) {
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
        allow_nxt[ct] = p.allowed[p.allowed_ls * layer + static_cast<int64_t>(min(tcol[ct], p.tq - 1)) * p.n_hist + g.u];
    }
  };
  auto finish_stage = [&](const Seg& g, char* buf) {
    __builtin_amdgcn_s_waitcnt(0);   // the asynchronous copies have landed
    __syncthreads();
    if (FMT != NKV_KV_BF16 && g.type == kSegHist) {
      dequant_i8<FMT>(p, g, lh, buf, tid);
      __syncthreads();
    }
  };

  // this tile's selected history blocks (per-query-tile selection: the ids
  // of the selection tile holding the workgroup's tokens)
  const int32_t* ids_row = p.ids + static_cast<int64_t>(layer) * p.ids_ls +
                           (p.sel_tile > 0 ? static_cast<int64_t>(t0 / p.sel_tile) * p.ids_tile_ls : 0);
  // the next segment at or after s that attends anything (its block id in
  // *blk): history ids outside [0, cap) (a union padded with -1) are passed
  // over, never staged
  auto next_seg = [&](int s, int* blk) {
    *blk = 0;
    for (; s < p.n_hist; ++s) {
      *blk = ids_row[s];
      if (*blk >= 0 && *blk < p.cap) break;
    }
    return s;
  };

  int blk_first;
  const int s_first = next_seg(seg_lo, &blk_first);
  Seg nxt = make_seg_blk<FMT>(p, layer, h, s_first < nseg ? s_first : 0, blk_first);
  if (s_first < nseg) {   // uniform: a split may have nothing left to attend
    begin_stage(nxt, lds0);
    finish_stage(nxt, lds0);
  }

  // One segment: compute on buffer P while the next segment is staged into
  // buffer 1 - P.
  // Returns the segment after s.
  auto step = [&](auto parity, int s) {
    constexpr int P = decltype(parity)::value;
    char* buf = P == 0 ? lds0 : lds1;
    char* other = P == 0 ? lds1 : lds0;
    const Seg cur = nxt;
    const int allow_cur[2] = {allow_nxt[0], allow_nxt[1]};
    int blk_next;
    const int s_next = next_seg(s + 1, &blk_next);
    const bool more = s_next < nseg;
    if (more) {
      nxt = make_seg_blk<FMT>(p, layer, h, s_next, blk_next);
      begin_stage(nxt, other);
    }

    // ---- S^T = K . Q^T -----------------------------------------------------
    f32x4 S[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) S[kt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(buf + kt * 4096 + koff[ks]);
        S[kt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[0][ks], S[kt][0], 0, 0, 0);
        S[kt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[1][ks], S[kt][1], 0, 0, 0);
      }
    }
    if (needs_mask<PACKED>(p, cur, t0)) apply_mask<PACKED>(p, cur, lg, tcol, allow_cur, S);

    // ---- online softmax (fp32) ----------------------------------------------
    float alpha[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      float mx = S[0][ct][0];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, S[kt][ct][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // the reference max only moves when a logit exceeds it by more than
      // 2^8 (p <= 256 is harmless in fp32 and bf16), so the accumulator
      // rescale below is rare
      const float cand = mx * p.scale_log2;
      const float m_new = cand > m_run[ct] + 8.0f ? cand : m_run[ct];
      const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
      alpha[ct] = __builtin_amdgcn_exp2f(m_run[ct] - m_use);
      m_run[ct] = m_new;
      float ls = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(S[kt][ct][e], p.scale_log2, -m_use));
          S[kt][ct][e] = pe;
          ls += pe;
        }
      l_run[ct] = l_run[ct] * alpha[ct] + ls;
    }
    if (__any(alpha[0] != 1.0f || alpha[1] != 1.0f)) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) acc[dt][ct] *= alpha[ct];
    }

    // ---- O^T += V^T . P^T ---------------------------------------------------
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      bf16x8 bp[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const f32x4 a0 = S[2 * k2][ct];
        const f32x4 a1 = S[2 * k2 + 1][ct];
        bp[ct] = __builtin_bit_cast(bf16x8, u32x4{pack_bf16(a0[0], a0[1]), pack_bf16(a0[2], a0[3]),
                                                  pack_bf16(a1[0], a1[1]), pack_bf16(a1[2], a1[3])});
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const char* vp = buf + vtr[dt & 3] + (dt >> 2) * 128 + k2 * 8192;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp + 4096));
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        acc[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[0], acc[dt][0], 0, 0, 0);
        acc[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[1], acc[dt][1], 0, 0, 0);
      }
    }

    if (more)
      finish_stage(nxt, other);
    else
      __syncthreads();
    return s_next;
  };

  for (int s = s_first; s < nseg;) {
    s = step(std::integral_constant<int, 0>{}, s);
    if (s < nseg) s = step(std::integral_constant<int, 1>{}, s);
  }

  // ---- normalise and store: acc[dt][ct][i] = dim 16 dt + 4 lg + i -----------
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    float l = l_run[ct];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const int t = tcol[ct];
    if (p.splits > 1) {
      // this split's (m, l, acc) of the column, merged by prefill_merge_kernel
      if (t <= t_last) {
        const int col = wave * 32 + ct * 16 + ln;
        float* rec = p.partial +
                     ((((static_cast<int64_t>(layer) * p.hkv + h) * nqt + qt) * p.splits + split) * kPfCols + col) *
                         kPfPart;
        if (lg == 0) {
          rec[0] = m_run[ct];
          rec[1] = l;
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(rec + 4 + 16 * dt + 4 * lg) = acc[dt][ct];
      }
    } else if (t <= t_last) {
      const float inv = 1.0f / l;
      uint16_t* orow = p.out + p.q_ls * layer + (static_cast<int64_t>(t) * hq + hcol[ct]) * kHeadDim + 4 * lg;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const f32x4 o = acc[dt][ct];
        *reinterpret_cast<u32x2*>(orow + 16 * dt) = u32x2{pack_bf16(o[0] * inv, o[1] * inv), pack_bf16(o[2] * inv, o[3] * inv)};
      }
    }
  }
}

// Merge the split partials of one (layer, KV head, query tile, column): one
// thread per dim, the usual rescale of each split's (m, l, acc) to the
// largest reference max.
__global__ __launch_bounds__(kHeadDim) void prefill_merge_kernel(const AttendParams p, int nqt) {
  const int h = blockIdx.x % p.hkv;
  const int qt = blockIdx.x / p.hkv;
  const int layer = blockIdx.y;
  const int col = blockIdx.z;
  const int t = qt * (kPfCols / p.G) + col / p.G;
  if (t >= p.tq) return;
  const int d = threadIdx.x;
  const int64_t sstride = static_cast<int64_t>(kPfCols) * kPfPart;
  const float* base =
      p.partial + (((static_cast<int64_t>(layer) * p.hkv + h) * nqt + qt) * p.splits * kPfCols + col) * kPfPart;
  float mt = -INFINITY;
  for (int s = 0; s < p.splits; ++s) mt = fmaxf(mt, base[s * sstride]);
  float L = 0.0f, A = 0.0f;
  for (int s = 0; s < p.splits; ++s) {
    const float* r = base + s * sstride;
    const float sw = (r[0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(r[0] - mt);
    L += r[1] * sw;
    A += r[4 + d] * sw;
  }
  const int hh = h * p.G + col % p.G;
  p.out[p.q_ls * layer + (static_cast<int64_t>(t) * p.hkv * p.G + hh) * kHeadDim + d] = f32_to_bf16(A / L);
}

}  // namespace

// The matrix-core kernel over (query tile x KV head, layer, split), then the
// split merge.
int launch_prefill(int hkv, int kv_format, int num_layers, int tq, AttendParams& p, hipStream_t s) {
  NKV_CHECK_SUPPORTED(p.G >= 1 && kPfCols % p.G == 0,
                      "nkv_prefill_attend: query heads per KV head (%d) must divide %d", p.G, kPfCols);
  const int tpw = kPfCols / p.G;
  const int nqt = (tq + tpw - 1) / tpw;
  const dim3 grid(nqt * hkv, num_layers, p.splits);
  const bool packed = p.tok_mask != nullptr || p.causal_off != 0;
  NKV_CHECK_SUPPORTED(!packed || kv_format == NKV_KV_BF16, "nkv_prefill_attend: caller-packed keys must be bf16");
  switch (kv_format) {
    case NKV_KV_BF16:
      if (packed)
        hipLaunchKernelGGL((prefill_kernel<NKV_KV_BF16, true>), grid, dim3(kPfThreads), 0, s, p, nqt);
      else
        hipLaunchKernelGGL((prefill_kernel<NKV_KV_BF16, false>), grid, dim3(kPfThreads), 0, s, p, nqt);
      break;
    case NKV_KV_INT8_CHANNEL:
      hipLaunchKernelGGL((prefill_kernel<NKV_KV_INT8_CHANNEL, false>), grid, dim3(kPfThreads), 0, s, p, nqt);
      break;
    case NKV_KV_INT8_TOKEN:
      hipLaunchKernelGGL((prefill_kernel<NKV_KV_INT8_TOKEN, false>), grid, dim3(kPfThreads), 0, s, p, nqt);
      break;
    default: NKV_CHECK_SUPPORTED(false, "nkv_prefill_attend: unknown kv_format %d", kv_format);
  }
  if (p.splits > 1)
    hipLaunchKernelGGL(prefill_merge_kernel, dim3(nqt * hkv, num_layers, min(kPfCols, tq * p.G)), dim3(kHeadDim), 0,
                       s, p, nqt);
  return NKV_OK;
}

}  // namespace nkv

using namespace nkv;

extern "C" int64_t nkv_prefill_workspace_floats(int num_layers, int num_kv_heads, int num_heads, int tq,
                                                int splits) {
  if (num_layers < 1 || num_kv_heads < 1 || num_heads < num_kv_heads || num_heads % num_kv_heads != 0 ||
      tq < 1 || splits < 1)
    return 0;
  const int G = num_heads / num_kv_heads;
  if (kPfCols % G != 0) return 0;
  const int64_t nqt = (tq + kPfCols / G - 1) / (kPfCols / G);
  return splits == 1 ? 0 : static_cast<int64_t>(num_layers) * num_kv_heads * nqt * splits * kPfCols * kPfPart;
}

extern "C" int nkv_prefill_attend(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                                  int64_t q_layer_stride, int tq, const uint16_t* k_new,
                                  const uint16_t* v_new, int64_t kv_layer_stride, const int32_t* ids,
                                  int64_t ids_layer_stride, int n_hist, const uint8_t* allowed,
                                  int64_t allowed_layer_stride, int sink_len, int ring_base, int rec_lo,
                                  int rec_len, float scale, int splits, float* partial_ws, uint16_t* out,
                                  void* stream) {
  AttendParams p;
  const int rc = fill_attend_params("nkv_prefill_attend", st, layer0, num_layers, q, q_layer_stride, tq,
                                    k_new, v_new, kv_layer_stride, tq, -1, ids, ids_layer_stride, n_hist,
                                    allowed, allowed_layer_stride, sink_len, ring_base, rec_lo, rec_len,
                                    scale, splits, partial_ws, out, &p);
  if (rc != NKV_OK) return rc;
  const int lrc = launch_prefill(st->num_kv_heads, st->kv_format, num_layers, tq, p,
                                 reinterpret_cast<hipStream_t>(stream));
  return lrc != NKV_OK ? lrc : launch_status("nkv_prefill_attend");
}

extern "C" int nkv_prefill_attend_tiled(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                                        int64_t q_layer_stride, int tq, const uint16_t* k_new, const uint16_t* v_new,
                                        int64_t kv_layer_stride, const int32_t* ids, int64_t ids_layer_stride,
                                        int64_t ids_tile_stride, int sel_tile, int n_hist, int sink_len, int ring_base,
                                        int rec_lo, int rec_len, float scale, int splits, float* partial_ws,
                                        uint16_t* out, void* stream) {
  AttendParams p;
  const int rc = fill_attend_params("nkv_prefill_attend_tiled", st, layer0, num_layers, q, q_layer_stride, tq, k_new,
                                    v_new, kv_layer_stride, tq, -1, ids, ids_layer_stride, n_hist, nullptr, 0,
                                    sink_len, ring_base, rec_lo, rec_len, scale, splits, partial_ws, out, &p);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_SUPPORTED(p.G >= 1 && kPfCols % p.G == 0,
                      "nkv_prefill_attend_tiled: query heads per KV head (%d) must divide %d", p.G, kPfCols);
  const int tpw = kPfCols / p.G;
  NKV_CHECK_ARG(sel_tile >= tpw && sel_tile % tpw == 0,
                "nkv_prefill_attend_tiled: sel_tile %d must be a positive multiple of the %d-token query tile",
                sel_tile, tpw);
  const int ntiles = (tq + sel_tile - 1) / sel_tile;
  NKV_CHECK_ARG(ids_tile_stride >= n_hist && ids_layer_stride >= static_cast<int64_t>(ntiles) * ids_tile_stride,
                "nkv_prefill_attend_tiled: id strides too small (tile %lld, layer %lld for %d tiles of %d ids)",
                static_cast<long long>(ids_tile_stride), static_cast<long long>(ids_layer_stride), ntiles, n_hist);
  p.ids_tile_ls = ids_tile_stride;
  p.sel_tile = sel_tile;
  const int lrc = launch_prefill(st->num_kv_heads, st->kv_format, num_layers, tq, p,
                                 reinterpret_cast<hipStream_t>(stream));
  return lrc != NKV_OK ? lrc : launch_status("nkv_prefill_attend_tiled");
}
