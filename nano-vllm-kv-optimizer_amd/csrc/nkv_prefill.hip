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
// Work split: one workgroup (4 wavefronts, two per CU) per (layer, KV head,
// query tile).  A query tile is 64 NCT columns = 64 NCT / G tokens x the G
// query heads of the KV head, so every K/V tile staged in LDS serves all G
// heads; wavefront w owns NCT 16-column MFMA tiles.  NCT = 3 (192 columns)
// for long chunks: each staged tile then feeds 1.5x the products of NCT = 2
// (128 columns, kept for short chunks, verify's per-query history flags and
// selection tiles 192 columns do not divide).  Workgroups are ordered so that
// the linear id cycles over the KV heads (one head per XCD when Hkv = 8,
// keeping that head's keys in one L2) and the longest causal tiles start
// first.
//
// Per 64-key segment (double-buffered LDS, one barrier per segment):
//   * staging: rows go global -> LDS directly (buffer_load ... lds issued as
//     inline assembly, no registers; bounds-checked descriptors read rows
//     past the segment as zero, so no index is clamped).  int8 history rows
//     land raw with their scales and are dequantised to bf16 in LDS after the
//     copy.  The next segment is in flight while the current one is computed;
//   * attend_segment: S^T = K . Q^T and O^T += V^T . P^T on the matrix cores
//     with an online softmax in between (its comment has the operand layout),
//     in one pass over the 64 keys (NCT = 2) or two of 32 (NCT = 3, half the
//     logits live).
//
// The reference runs this as flash-attention over the packed
// [selected | sink | recent | chunk] keys with bottom-right causal masking
// (nanovllm/sparse/m12_runtime.py:592-651, :809-839); the fp32 masked path
// (:875-896) is the same function.
#include <algorithm>
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

// Workgroup barrier that drains this wavefront's LDS operations only: the
// asynchronous global -> LDS copies stay in flight (__syncthreads' fence would
// wait for every outstanding vector-memory operation, copies included).  The
// memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt untouched
  asm volatile("s_barrier" ::: "memory");
}

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

// bf16 segment -> stage buffer with WAVES wavefronts: wavefront w copies K and
// V rows (64 / WAVES) w .. + 64 / WAVES, four rows (1 KiB) per instruction;
// lane u lands at 16 u of its 1 KiB, so it fetches the global chunk that the
// swizzle puts there.  Whole offsets go in the bounds-checked lane offset.
template <int WAVES>
__device__ __forceinline__ void dma_rows(const Seg& g, char* buf, int wave, int lane, bool live) {
  constexpr int RPW = kBlock / WAVES;
  const uint32_t bytes = live ? static_cast<uint32_t>(g.len * g.rowb) : 0u;
  const rsrc_words rk = rsrc_of(g.kbase, bytes);
  const rsrc_words rv = rsrc_of(g.vbase, bytes);
  const int ln = lane & 15;
  const int lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < RPW / 4; ++i) {
    const int row = RPW * wave + 4 * i + lg;
    const char* dst = buf + (RPW * wave + 4 * i) * 256;
    lds_copy16(rk, dst, row * g.rowb + ((ln ^ (row & 15)) << 4));
    lds_copy16(rv, dst + kTileBytes, row * g.rowb + ((ln ^ (2 * lg)) << 4));
  }
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

template <int FMT, int WAVES = 4>
__device__ __forceinline__ void dma_i8_segment(const AttendParams& p, const Seg& g, int lh, char* buf, int wave,
                                               int lane, bool live = true) {
  const uint32_t bytes = live ? static_cast<uint32_t>(g.len * g.rowb) : 0u;
  const rsrc_words rk = rsrc_of(g.kbase, bytes);
  const rsrc_words rv = rsrc_of(g.vbase, bytes);
  constexpr int kPer = 8 / WAVES;   // 1 KiB copies per tensor and wavefront
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int o = (kPer * wave + i) * 1024;
    lds_copy16(rk, buf + kI8RawK + o, o + lane * 16);
    lds_copy16(rv, buf + kI8RawV + o, o + lane * 16);
  }
  if (wave == 0) {
    if (FMT == NKV_KV_INT8_TOKEN) {
      // 64 fp16 scales = 128 B per tensor; lanes 32.. read past it (zeros)
      const int64_t tb = (static_cast<int64_t>(lh) * p.cap + g.blk) * kBlock;
      lds_copy4(rsrc_of(p.k_tscale + tb, kBlock * 2), buf + kI8Scales, lane * 4);
      lds_copy4(rsrc_of(p.v_tscale + tb, kBlock * 2), buf + kI8VScales, lane * 4);
    } else {
      // 128 fp32 per-(head, dim) K scales
      const rsrc_words sk = rsrc_of(p.k_scale + static_cast<int64_t>(lh) * kHeadDim, kHeadDim * 4);
      lds_copy4(sk, buf + kI8Scales, lane * 4);
      lds_copy4(sk, buf + kI8Scales + 256, 256 + lane * 4);
    }
  }
}

// In-place dequantisation of a staged int8 block (the copies have landed and
// are visible): with NT threads, thread tid converts rows (tid >> 4) + (NT / 16) j,
// dims 8 c .. 8 c + 7 (c = tid & 15) of K and V to bf16(code * scale) in the
// K / V tiles.
template <int FMT, int NT = kPfThreads>
__device__ __forceinline__ void dequant_i8(const AttendParams& p, const Seg& g, int lh, char* buf, int tid) {
  constexpr int RS = NT / 16;        // row step
  constexpr int NJ = kBlock / RS;    // rows per thread
  const int r0 = tid >> 4;
  const int c = tid & 15;
  u32x2 kq[NJ], vq[NJ];
  float ksc[NJ][8], vsc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int r = r0 + RS * j;
    kq[j] = *reinterpret_cast<const u32x2*>(buf + kI8RawK + r * kHeadDim + c * 8);
    vq[j] = *reinterpret_cast<const u32x2*>(buf + kI8RawV + r * kHeadDim + c * 8);
  }
  if (FMT == NKV_KV_INT8_TOKEN) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int r = r0 + RS * j;
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
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ksc[j][e] = __uint_as_float(s0[e]);
        ksc[j][e + 4] = __uint_as_float(s1[e]);
      }
      vsc[j] = vs;
    }
  }
  lds_barrier();   // every raw code and scale has been read
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int r = r0 + RS * j;
    float vv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vv[e] = vsc[j];
    *reinterpret_cast<u32x4*>(buf + r * 256 + ((c ^ (r0 & 15)) << 4)) = dequant8(kq[j][0], kq[j][1], ksc[j]);
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
template <bool PACKED, int NCT, int KT>
__device__ __forceinline__ void apply_mask(const AttendParams& p, const Seg& g, int lg, const int (&tcol)[NCT],
                                           const int (&allow)[NCT], f32x4 (&S)[KT][NCT], int kt0) {
  if (g.type == kSegRecent) {
    // x = (slot - ring_base - rec_lo) mod R for slot off + key
    int a = (g.off - p.ring_base - p.rec_lo) % p.R;
    a = a < 0 ? a + p.R : a;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 16 * (kt0 + kt) + 4 * lg + e;
        int x = a + key;
        x -= p.R & ((p.R - 1 - x) >> 31);
        const float bound = vis_bound(max(key - (g.vlen - 1), x - (p.rec_len - 1)));
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) S[kt][ct][e] = fminf(S[kt][ct][e], bound);
      }
    return;
  }
  int base[NCT];   // 4 lg - thr[ct]
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    int thr = g.vlen - 1;
    if (g.type == kSegChunk) thr = min(thr, tcol[ct] + (PACKED ? p.causal_off : 0) - g.off);
    else if (allow[ct] == 0) thr = -1;
    base[ct] = 4 * lg - thr;
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[kt][ct][e] = fminf(S[kt][ct][e], vis_bound(base[ct] + 16 * (kt0 + kt) + e));
  if (PACKED && g.type == kSegChunk && p.tok_mask != nullptr) {
    // caller-packed keys with a per-(query, key) mask: keys past vlen are
    // already hidden and never read; padding columns read row tq - 1
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const uint8_t* mrow = p.tok_mask + static_cast<int64_t>(min(tcol[ct], p.tq - 1)) * p.n_chunk + g.off;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = 16 * (kt0 + kt) + 4 * lg + e;
          if (key < g.vlen && mrow[key] != 0) S[kt][ct][e] = -INFINITY;
        }
    }
  }
}

// Loop-invariant LDS offsets (bytes) of a lane's MFMA operands in a stage
// buffer.  K read (QK A operand): key 16 kt + ln, 16-byte chunk 4 ks + lg,
// at koff[ks] + 4096 kt.  V transposing read (PV A operand): lane ln
// addresses key 4 lg + (ln >> 2) (+ 32 k2 + 16 half), dims 16 dt + 4 (ln & 3)
// .. +4; the swizzled chunk is 2 (dt ^ (ln >> 2)) + ((ln & 3) >> 1), so
// dt & 4 -> + 128 and dt & 3 picks vtr[].
struct OperandOffsets {
  int koff[4];
  int vtr[4];
  __device__ __forceinline__ OperandOffsets(int ln, int lg) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) koff[ks] = ln * 256 + ((((4 * ks + lg) ^ ln) & 15) << 4);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      vtr[q] = kTileBytes + (4 * lg + (ln >> 2)) * 256 + ((2 * (q ^ (ln >> 2)) + ((ln & 3) >> 1)) << 4) + 8 * (ln & 1);
  }
};

// Online-softmax state of one column: the reference max in log2 units is
// -nm (nm = 0 and thr = -inf before any key was visible); a logit above thr
// (raw units) would move it by more than 2^8; l is the running denominator.
struct Col {
  float nm;
  float thr;
};
__device__ __forceinline__ void col_init(Col& c) {
  c.nm = 0.0f;
  c.thr = -INFINITY;
}
__device__ __forceinline__ float col_max(const Col& c) { return c.thr == -INFINITY ? -INFINITY : -c.nm; }

// One staged segment (64 keys in `buf`) against the wavefront's NCT 16-column
// tiles, in passes of 16 KT keys (KT = 4: one pass; KT = 2: two passes with
// half the logits live):
//   * S^T = K . Q^T: v_mfma_f32_16x16x32_bf16, A = 16 keys x 32 dims read
//     from the K tile, B = 32 dims x 16 columns held in registers (bq);
//   * the visibility mask when `mask`;
//   * online softmax in fp32 per column (exp2, scale folded in; the running
//     max and the rescale stay in the lane, whose column is fixed);
//   * O^T += V^T . P^T: A = 16 dims x 32 keys from two transposing LDS reads
//     (ds_read_b64_tr_b16), B = the lane's own probabilities rounded to bf16
//     (the 32-key contraction index is ordered as the S^T accumulator holds
//     the keys, so P never leaves the registers); the row sums l are one
//     more product per 32 keys, of the same bf16-rounded P with a constant
//     all-ones A operand (every accumulator row holds the column's sum), so
//     numerator and denominator see the same P.
template <bool PACKED, int NCT, int KT>
__device__ __forceinline__ void attend_segment(const AttendParams& p, const Seg& cur, const char* buf, bool mask,
                                               int lg, const OperandOffsets& off, const bf16x8 (&bq)[NCT][4],
                                               const int (&tcol)[NCT], const int (&allow)[NCT],
                                               f32x4 (&acc)[8][NCT], f32x4 (&lsum)[NCT], Col (&col)[NCT]) {
  // Operand reads run two products ahead through a ring of three registers;
  // the scheduling barriers keep that order (left to itself the scheduler may
  // sink each read onto its product and wait out the full LDS latency).
  constexpr int kQ = 4 * KT;   // K operands per pass: ks outer, kt inner
  auto read_k = [&](int pass, int i) {
    return *reinterpret_cast<const bf16x8*>(buf + (pass * KT + i % KT) * 4096 + off.koff[i / KT]);
  };
  auto read_v = [&](int k2, int dt) {
    const char* vp = buf + off.vtr[dt & 3] + (dt >> 2) * 128 + k2 * 8192;
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp + 4096));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };
#pragma unroll
  for (int pass = 0; pass < 4 / KT; ++pass) {
    // ---- S^T = K . Q^T ---------------------------------------------------
    f32x4 S[KT][NCT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) S[kt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 ka[3];
    ka[0] = read_k(pass, 0);
    ka[1] = read_k(pass, 1);
#pragma unroll
    for (int i = 0; i < kQ; ++i) {
      if (i + 2 < kQ) ka[(i + 2) % 3] = read_k(pass, i + 2);
      const int ks = i / KT;
      const int kt = i % KT;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        S[kt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[i % 3], bq[ct][ks], S[kt][ct], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the first V operands load while the softmax runs
    const int k2_0 = pass * (KT / 2);
    bf16x8 va[3];
    va[0] = read_v(k2_0, 0);
    va[1] = read_v(k2_0, 1);
    __builtin_amdgcn_sched_barrier(0);
    if (mask) {
      // (an empty volatile asm: the compiler would otherwise compute the
      // branch-free mask on every segment, though few need one)
      asm volatile("");
      apply_mask<PACKED, NCT, KT>(p, cur, lg, tcol, allow, S, pass * KT);
    }

    // ---- online softmax (fp32) --------------------------------------------
    // The reference max only moves when a logit exceeds it by more than 2^8
    // (p <= 256 is harmless in fp32 and bf16): each lane compares its own
    // logits with the column's threshold, and only when some column of the
    // wavefront crosses it (always on a column's first visible keys) are the
    // column maxima reduced across lanes and the accumulators rescaled.
    float mx[NCT];
    bool move = false;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      mx[ct] = S[0][ct][0];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) mx[ct] = fmaxf(mx[ct], S[kt][ct][e]);
      move = move || mx[ct] > col[ct].thr;
    }
    if (__any(move)) {
      asm volatile("");
      float alpha[NCT];
      bool rescale = false;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const float m_old = col_max(col[ct]);
        const float cand = max_over_rows(mx[ct]) * p.scale_log2;
        const float m_new = cand > m_old + 8.0f ? cand : m_old;
        const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
        alpha[ct] = __builtin_amdgcn_exp2f(m_old - m_use);
        rescale = rescale || alpha[ct] != 1.0f;
        col[ct].nm = -m_use;
        col[ct].thr = m_new == -INFINITY ? -INFINITY : (m_new + 8.0f) / p.scale_log2;
        lsum[ct] *= alpha[ct];
      }
      if (__any(rescale)) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) acc[dt][ct] *= alpha[ct];
      }
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          S[kt][ct][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[kt][ct][e], p.scale_log2, col[ct].nm));

    // ---- O^T += V^T . P^T -------------------------------------------------
    constexpr int kV = 8 * (KT / 2);   // V operands per pass: 32-key group outer, dt inner
#pragma unroll
    for (int i = 0; i < kV; ++i) {
      const int j = i / 8;
      const int dt = i % 8;
      if (dt == 0) __builtin_amdgcn_sched_barrier(0);
      bf16x8 bp[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const f32x4 a0 = S[2 * j][ct];
        const f32x4 a1 = S[2 * j + 1][ct];
        const u32x4 w = u32x4{pack_bf16(a0[0], a0[1]), pack_bf16(a0[2], a0[3]), pack_bf16(a1[0], a1[1]),
                              pack_bf16(a1[2], a1[3])};
        bp[ct] = __builtin_bit_cast(bf16x8, w);
        if (dt == 0) {
          const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
          lsum[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, bp[ct], lsum[ct], 0, 0, 0);
        }
      }
      if (i + 2 < kV) va[(i + 2) % 3] = read_v(k2_0 + (i + 2) / 8, (i + 2) % 8);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc[dt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[i % 3], bp[ct], acc[dt][ct], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// PACKED: caller-packed keys (nkv_attend_packed): the chunk's causal start is
// causal_off and an optional per-token mask applies; its own instantiation,
// so the history paths carry none of that code.
template <int FMT, bool PACKED, int NCT>
__global__ __launch_bounds__(kPfThreads, 2) void prefill_kernel(const AttendParams p, int nqt) {
  constexpr int kCols = kPfWaves * 16 * NCT;   // (token, head) columns per workgroup
  // per-query history flags (verify's union selections) take the 128-column
  // tiling only: the wider one keeps those registers for its logits
  constexpr bool kAllowed = NCT == 2;
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
  const int tpw = kCols / p.G;
  const int t0 = qt * tpw;
  const int t_last = min(t0 + tpw, p.tq) - 1;
  const int hq = p.hkv * p.G;

  const OperandOffsets off(ln, lg);

  // ---- query operands: column c = 16 NCT wave + 16 ct + ln ----------------
  bf16x8 bq[NCT][4];
  int tcol[NCT];
  // the column's query head (recomputed for the store: no register held)
  auto head_of = [&](int ct) { return h * p.G + (wave * 16 * NCT + ct * 16 + ln) % p.G; };
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int c = wave * 16 * NCT + ct * 16 + ln;
    const int t = t0 + c / p.G;
    tcol[ct] = t;
    const uint16_t* qrow = p.q + p.q_ls * layer + (static_cast<int64_t>(t) * hq + head_of(ct)) * kHeadDim + lg * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (t < p.tq) v = *reinterpret_cast<const u32x4*>(qrow + ks * 32);
      bq[ct][ks] = __builtin_bit_cast(bf16x8, v);
    }
  }

  f32x4 acc[8][NCT];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[dt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  f32x4 lsum[NCT];   // row sums: every row of a column's accumulator holds its sum
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) lsum[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  Col cs[NCT];   // per-column softmax state
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) col_init(cs[ct]);

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
  int allow_nxt[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) allow_nxt[ct] = 1;
  auto begin_stage = [&](const Seg& g, char* buf) {
    // the column flags are loaded before the copies: vector memory counts
    // complete in order, so waiting for the flags then leaves the copies in
    // flight (issued after them, the flags' wait would drain the copies too)
    if (kAllowed && g.type == kSegHist && p.allowed != nullptr) {
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        allow_nxt[ct] = p.allowed[p.allowed_ls * layer + static_cast<int64_t>(min(tcol[ct], p.tq - 1)) * p.n_hist + g.u];
    }
    if (FMT != NKV_KV_BF16 && g.type == kSegHist)
      dma_i8_segment<FMT>(p, g, lh, buf, wave, lane);
    else
      dma_rows<kPfWaves>(g, buf, wave, lane, true);
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
  // (read through the constant address space: scalar loads, counted by
  // lgkmcnt -- a vector load here would be waited for with vmcnt(0) before
  // the next segment's copies could issue)
  typedef __attribute__((address_space(4))) const int32_t cint32;
  const cint32* ids_row = (const cint32*)(p.ids + static_cast<int64_t>(layer) * p.ids_ls +
                                          (p.sel_tile > 0 ? static_cast<int64_t>(t0 / p.sel_tile) * p.ids_tile_ls : 0));
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
    int allow_cur[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) allow_cur[ct] = allow_nxt[ct];
    int blk_next;
    const int s_next = next_seg(s + 1, &blk_next);
    const bool more = s_next < nseg;
    if (more) {
      nxt = make_seg_blk<FMT>(p, layer, h, s_next, blk_next);
      begin_stage(nxt, other);
    }

    attend_segment<PACKED, NCT, NCT == 2 ? 4 : 2>(p, cur, buf, needs_mask<PACKED>(p, cur, t0), lg, off, bq, tcol,
                                                 allow_cur, acc, lsum, cs);

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
  for (int ct = 0; ct < NCT; ++ct) {
    const float l = lsum[ct][0];
    const int t = tcol[ct];
    if (p.splits > 1) {
      // this split's (m, l, acc) of the column, merged by prefill_merge_kernel
      if (t <= t_last) {
        const int col = wave * 16 * NCT + ct * 16 + ln;
        float* rec = p.partial +
                     ((((static_cast<int64_t>(layer) * p.hkv + h) * nqt + qt) * p.splits + split) * kCols + col) *
                         kPfPart;
        if (lg == 0) {
          rec[0] = col_max(cs[ct]);
          rec[1] = l;
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(rec + 4 + 16 * dt + 4 * lg) = acc[dt][ct];
      }
    } else if (t <= t_last) {
      const float inv = 1.0f / l;
      uint16_t* orow = p.out + p.q_ls * layer + (static_cast<int64_t>(t) * hq + head_of(ct)) * kHeadDim + 4 * lg;
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
__global__ __launch_bounds__(kHeadDim) void prefill_merge_kernel(const AttendParams p, int nqt, int cols) {
  const int h = blockIdx.x % p.hkv;
  const int qt = blockIdx.x / p.hkv;
  const int layer = blockIdx.y;
  const int col = blockIdx.z;
  const int t = qt * (cols / p.G) + col / p.G;
  if (t >= p.tq) return;
  const int d = threadIdx.x;
  const int64_t sstride = static_cast<int64_t>(cols) * kPfPart;
  const float* base =
      p.partial + (((static_cast<int64_t>(layer) * p.hkv + h) * nqt + qt) * p.splits * cols + col) * kPfPart;
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

// Columns per workgroup a launch takes: 192 (three 16-column tiles per
// wavefront: each staged K / V tile serves 1.5x the columns, for 1.5x fewer
// LDS reads per product) when G divides it, the selection tile (if any) is a
// whole number of its token tiles and the chunk fills two of them; 128
// otherwise.  Per-query history flags keep the 128-column kernel, which holds
// them in registers the wider one spends on its logits.
int prefill_cols(const AttendParams& p, int tq) {
  constexpr int kWide = 3 * 64;
  if (kWide % p.G != 0 || p.allowed != nullptr) return kPfCols;
  if (p.sel_tile > 0 && p.sel_tile % (kWide / p.G) != 0) return kPfCols;
  return static_cast<int64_t>(tq) * p.G >= 2 * kWide ? kWide : kPfCols;
}

template <int FMT, bool PACKED>
void launch_prefill_fmt(int cols, const dim3& grid, AttendParams& p, int nqt, hipStream_t s) {
  if (cols == kPfCols)
    hipLaunchKernelGGL((prefill_kernel<FMT, PACKED, 2>), grid, dim3(kPfThreads), 0, s, p, nqt);
  else
    hipLaunchKernelGGL((prefill_kernel<FMT, PACKED, 3>), grid, dim3(kPfThreads), 0, s, p, nqt);
}

// The matrix-core kernel over (query tile x KV head, layer, split), then the
// split merge.
int launch_prefill(int hkv, int kv_format, int num_layers, int tq, AttendParams& p, hipStream_t s) {
  NKV_CHECK_ARG(p.splits >= 1, "nkv_prefill_attend: splits must be in [1, 64] (got %d)", p.splits);
  NKV_CHECK_SUPPORTED(p.G >= 1 && kPfCols % p.G == 0,
                      "nkv_prefill_attend: query heads per KV head (%d) must divide %d", p.G, kPfCols);
  const int cols = prefill_cols(p, tq);
  const int tpw = cols / p.G;
  const int nqt = (tq + tpw - 1) / tpw;
  const dim3 grid(nqt * hkv, num_layers, p.splits);
  const bool packed = p.tok_mask != nullptr || p.causal_off != 0;
  NKV_CHECK_SUPPORTED(!packed || kv_format == NKV_KV_BF16, "nkv_prefill_attend: caller-packed keys must be bf16");
  switch (kv_format) {
    case NKV_KV_BF16:
      if (packed)
        launch_prefill_fmt<NKV_KV_BF16, true>(cols, grid, p, nqt, s);
      else
        launch_prefill_fmt<NKV_KV_BF16, false>(cols, grid, p, nqt, s);
      break;
    case NKV_KV_INT8_CHANNEL: launch_prefill_fmt<NKV_KV_INT8_CHANNEL, false>(cols, grid, p, nqt, s); break;
    case NKV_KV_INT8_TOKEN: launch_prefill_fmt<NKV_KV_INT8_TOKEN, false>(cols, grid, p, nqt, s); break;
    default: NKV_CHECK_SUPPORTED(false, "nkv_prefill_attend: unknown kv_format %d", kv_format);
  }
  if (p.splits > 1)
    hipLaunchKernelGGL(prefill_merge_kernel, dim3(nqt * hkv, num_layers, min(cols, tq * p.G)), dim3(kHeadDim), 0, s, p,
                       nqt, cols);
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
  if (kPfCols % G != 0 || splits == 1) return 0;
  // any tiling may run: the largest need
  int64_t cols_total = 0;
  for (int cols : {kPfCols, 3 * 64})
    if (cols % G == 0)
      cols_total = std::max<int64_t>(cols_total, ((tq + cols / G - 1) / (cols / G)) * static_cast<int64_t>(cols));
  return static_cast<int64_t>(num_layers) * num_kv_heads * splits * cols_total * kPfPart;
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
