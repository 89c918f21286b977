// Segmented GQA attention for few queries: sparse decode and speculative
// verify (kernel 3 of the layer-step).
//
// One workgroup (4 wavefronts) handles one (layer, KV head, query group,
// split).  The keys it attends are cut into segments of up to 64 rows that
// are contiguous in memory with a uniform row stride:
//   * the selected history blocks, read in place from the HBM history
//     (bf16 or int8),
//   * the sink,
//   * the recent ring, walked in physical 64-slot pieces; a slot takes part
//     when its logical position lies in the requested window,
//   * the chunk of new tokens (verify's Tq tokens, or decode's new token),
//     causal: query t sees chunk token c iff c <= t.
// Row indices are clamped into each segment, so every load stays inside its
// buffer; validity is applied as a -inf mask on the logits.  Split form:
// wavefront w of split s handles segments w + 4 s, w + 4 s + 4 splits, ...
// with an online softmax.  Stream form (4 query rows, decode): the launch is
// one resident round of wavefronts, the same number per (layer, KV head,
// group), each taking an equal run of its group's segments, so none waits
// at a workgroup merge; 36-layer 32K decode, bf16 attention 71.3 -> 68.4 us,
// int8 58.4 -> 51.6 us (the split form left the second, partly filled round
// of workgroups and each workgroup's slowest wavefront on the critical path:
// ~20-28% of wavefront time in prologue and merge waits).
// The wide few-query kernel (verify) keeps workgroups, which share the
// query operands in LDS; its splits-0 form is a tiered plan instead: the
// first groups in larger pieces filling one round of workgroups, the rest
// in pieces about 3/4 that size filling a second, which also back-fill the
// slots the slower first-round workgroups free late.
//
//  * Q.K^T runs on the matrix cores: v_mfma_f32_16x16x32_bf16 with A = 16
//    keys x 32 dims (each lane loads 16 contiguous bytes of one key row) and
//    B = 32 dims x 16 query rows (G heads per query, padded to 16).  int8
//    keys are widened to bf16 exactly; the per-(head, dim) K scale is folded
//    into the bf16 query operand of history segments.
//  * softmax: fp32, exp2 with the scale folded in.
//  * P.V, 4 query rows (decode): on the matrix cores.  V (int8 widened to
//    bf16 exactly) goes to the wave's LDS tile and is read back transposed
//    (ds_read_b64_tr_b16) as the A operand; P^T comes straight from the
//    Q.K^T output registers as bf16 hi + lo parts, so P.V keeps fp32
//    accuracy.  V loads are issued together with the K loads, so a
//    segment's 32 KiB (bf16) are in flight at once.
//  * P.V, 8 or 16 query rows (verify): on the vector ALUs in fp32: lane
//    (r, c) owns dims 8c..8c+7 of keys 4j + r; p comes from LDS.  V loads are
//    issued right after the MFMAs, overlapping the softmax.
//    In both forms the int8 V scale (per block or per token) is folded into p.
//  * split form: the 4 wavefronts merge through LDS; with splits > 1 each
//    workgroup writes a partial (m, l, acc[128]) per query row and a second
//    kernel merges them (stream order makes the partials visible).  Stream
//    form: each wavefront writes its own partial.
//
// Same result as the reference's gather + pack + fp32 einsum attention
// (nanovllm/sparse/m12_runtime.py:1212-1320 and :845-896) up to fp32
// summation order.
#include <algorithm>
#include <type_traits>

#include "nkv_attend_common.h"
#include "nkv_stage.h"

namespace nkv {
namespace {
using namespace attend_detail;

// LDS floats of one workgroup: the per-wave p tiles during the segment loop,
// reused afterwards for the cross-wave merge (m, l and acc of every wave).
template <int M>
constexpr int attend_lds_floats() {
  return kAttendWaves * kBlock * kPRow > 2 * kAttendWaves * kMaxRows + kAttendWaves * M * kHeadDim
             ? kAttendWaves * kBlock * kPRow
             : 2 * kAttendWaves * kMaxRows + kAttendWaves * M * kHeadDim;
}

// The 4-row (decode) variants run P.V on the matrix cores: the vector-ALU
// form costs 512 fp32 FMAs per lane and segment, which with the int8
// dequantisation no longer hides under the loads (36-layer 32K step: bf16
// attention 86.6 -> 83.2 us, int8 77.0 -> 74.2, int8 per-token 84.6 -> 79.2).
// The wider variants keep fp32 P.V on the vector ALUs (their accumulators
// would not fit beside the V tiles).
template <int FMT, int M>
constexpr bool attend_mfma_pv() {
  return M == 4;
}
constexpr int kVTileBytes = kBlock * kHeadDim * 2;   // one bf16 V tile in LDS
static_assert(2 * kAttendWaves * kMaxRows + kAttendWaves * 4 * kHeadDim <= kAttendWaves * kVTileBytes / 4,
              "the cross-wave merge fits in the V tiles");

// PACKED: caller-packed keys (nkv_attend_packed): the chunk's causal start is
// causal_off and an optional per-token mask applies; its own instantiation,
// so the decode and verify paths carry none of that code.
// STREAM: the stream form (see the end of the kernel); its own instantiation,
// so neither form carries the other's code.
template <int FMT, int M, bool PACKED, bool STREAM = false>
__global__ __launch_bounds__(kAttendThreads, M == 4 ? NKV_ATTEND_DECODE_WAVES : 1) void attend_kernel(const AttendParams p) {
  constexpr bool kMfmaPV = attend_mfma_pv<FMT, M>();
  __shared__ __attribute__((aligned(16))) float s_lds[kMfmaPV ? kAttendWaves * kVTileBytes / 4 : attend_lds_floats<M>()];
  __shared__ float s_alpha[kMfmaPV ? 1 : kAttendWaves][kMaxRows];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int ln = lane & 15;   // MFMA column / PV dim group
  const int lg = lane >> 4;   // MFMA row group / PV key residue
  const int hq = p.hkv * p.G;

  // One (layer, KV head, query group): this wavefront attends its segments
  // s_begin, s_begin + s_step, ... below s_end.  rec < 0 (split form): the
  // four wavefronts then merge in LDS and the workgroup writes the output or
  // its split partial; rec >= 0 (stream form): the wavefront writes its own
  // partial record rec.  `duties`: this workgroup (split form: split 0) or
  // wavefront (stream form: the one attending the group's first segment)
  // also clears the layer's score keys and appends the decode token.
  auto group = [&](const int layer, const int h, const int qg, const int s_begin, const int s_step, const int s_end,
                   const bool duties, const int rec) __attribute__((always_inline)) {
  constexpr bool stream = STREAM;
  const int q0 = qg * p.qpg;
  const int rows = min(p.qpg, p.tq - q0) * p.G;

  // The ring position: the call's, or this layer's ring start in device
  // memory (reduced mod R, so any stored value addresses a ring slot).
  int write_slot = p.write_slot, ring_base = p.ring_base;
  if (p.ring_start != nullptr) {
    write_slot = static_cast<int>(static_cast<uint32_t>(p.ring_start[layer]) % static_cast<uint32_t>(p.R));
    ring_base = write_slot + 1 == p.R ? 0 : write_slot + 1;
  }

  // the decode step's score keys: read by its top-k launch, cleared here for
  // the next step's scoring (stream order makes both safe)
  if (p.zero_keys != nullptr && duties && h == 0 && qg == 0) {
    uint32_t* zk = p.zero_keys + static_cast<int64_t>(layer) * p.zero_n;
    if (stream) {
      for (int i = lane; i < p.zero_n; i += kWave) zk[i] = 0u;
    } else {
      for (int i = threadIdx.x; i < p.zero_n; i += kAttendThreads) zk[i] = 0u;
    }
  }

  // decode's shift+append: the new token (chunk token 0) also goes into the
  // freed ring slot, which no workgroup of this launch reads.
  if (write_slot >= 0 && duties && qg == 0 && (stream || wave == 0) && lane < 32) {
    const int which = lane >> 4;
    const int c = lane & 15;
    const uint4* src = reinterpret_cast<const uint4*>(
        (which ? p.v_new : p.k_new) + p.kv_ls * layer + static_cast<int64_t>(h) * kHeadDim);
    uint4* dst = reinterpret_cast<uint4*>(
        (which ? p.rec_v : p.rec_k) + p.rec_ls * layer +
        (static_cast<int64_t>(h) * p.R + write_slot) * kHeadDim);
    dst[c] = src[c];
  }

  // ---- query operands (B of the MFMA): row n = lane & 15 -------------------
  const int my_row = ln;
  const bool row_ok = my_row < rows;
  const int my_t = q0 + (row_ok ? my_row / p.G : 0);
  const int my_hq = h * p.G + (my_row % p.G);
  bf16x8 bq[4], bqs[4];
  // int8 history segments take their keys as two 16-byte loads of 16
  // contiguous codes (dims [16 lg, +16) and [64 + 16 lg, +16) of a key row:
  // each load covers 64 contiguous bytes of 16 rows), so their MFMA step s
  // contracts dims [64 (s >> 1) + 16 lg + 8 (s & 1), +8): the int8 query
  // operand bqs covers those dims (the contraction is over all 128 dims
  // either way).  Its
  // loads (the query row, and for per-channel int8 the K scales of this
  // lane's dims) all issue before the scaled operands are formed: a
  // conversion between them would make each load a round trip of its own.
  // With int8 history the plain operand bq serves only the bf16 segments,
  // which run after the int8 ones: it is loaded then (load_bq), so its
  // registers are free during the int8 segments.
  const uint16_t* my_qrow = p.q + p.q_ls * layer + (static_cast<int64_t>(my_t) * hq + my_hq) * kHeadDim;
  auto load_bq = [&]() __attribute__((always_inline)) {
    uint4 qv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qv[s] = make_uint4(0u, 0u, 0u, 0u);
      if (row_ok) qv[s] = *reinterpret_cast<const uint4*>(my_qrow + s * 32 + lg * 8);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) bq[s] = as_bf16x8(qv[s]);
  };
  if (FMT == NKV_KV_BF16) load_bq();
  uint4 qp[4];
  float4 ksc[4][2];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int dp = (s >> 1) * 64 + lg * 16 + (s & 1) * 8;
    qp[s] = make_uint4(0u, 0u, 0u, 0u);
    if (FMT != NKV_KV_BF16 && row_ok) qp[s] = *reinterpret_cast<const uint4*>(my_qrow + dp);
    if (FMT == NKV_KV_INT8_CHANNEL) {
      const float4* ks = reinterpret_cast<const float4*>(
          p.k_scale + static_cast<int64_t>(layer) * p.hkv * kHeadDim + h * kHeadDim + dp);
      ksc[s][0] = ks[0];
      ksc[s][1] = ks[1];
    }
  }
  // the int8 operand bqs: formed by the wave's first int8 segment once its
  // key and value loads are in flight, so the wait for the query and scale
  // loads does not hold them back
  auto make_bqs = [&]() __attribute__((always_inline)) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint4 v = qp[s];
    if (FMT == NKV_KV_INT8_CHANNEL) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      const float sc[8] = {ksc[s][0].x, ksc[s][0].y, ksc[s][0].z, ksc[s][0].w,
                           ksc[s][1].x, ksc[s][1].y, ksc[s][1].z, ksc[s][1].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = bf16_lo(w[i]) * sc[2 * i];
        const float b = bf16_hi(w[i]) * sc[2 * i + 1];
        o[i] = static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
      }
      bqs[s] = as_bf16x8(make_uint4(o[0], o[1], o[2], o[3]));
    } else if (FMT != NKV_KV_BF16) {
      bqs[s] = as_bf16x8(v);
    }
  }
  };

  float m_run = -INFINITY;   // per query row (lane & 15); equal across lane groups
  float l_run = 0.0f;        // partial over this lane group's keys
  float acc[M][8];           // vector-ALU P.V: dims 8 ln .. +8 of row n, keys = lg mod 4
  f32x4 oacc[8];             // matrix-core P.V: O^T, oacc[dt][i] = dim 16 dt + 4 lg + i of row ln
#pragma unroll
  for (int n = 0; n < M; ++n)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[n][e] = 0.0f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) oacc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  float* my_p = s_lds + wave * kBlock * kPRow;
  // matrix-core P.V: this wave's V tile in LDS, key-major with chunk c of key
  // k at position c ^ 2 (k & 3); V register (key 4 j + lg, chunk ln) lands at
  // j * 1024 + vw.  The transposing reads (ds_read_b64_tr_b16) give lane ln
  // keys 4 lg + (ln >> 2) (+ 32 k2, + 16 for the high half), dims 16 dt +
  // 4 (ln & 3) + 0..3; vtr[dt & 3] is that lane's offset, dt & 4 adds 128.
  char* my_v = reinterpret_cast<char*>(s_lds) + wave * kVTileBytes;
  const int vw = lg * 256 + ((ln ^ (2 * lg)) << 4);
  int vtr[4];
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4)
    vtr[q4] = (4 * lg + (ln >> 2)) * 256 + ((2 * (q4 ^ (ln >> 2)) + ((ln & 3) >> 1)) << 4) + 8 * (ln & 1);
  // History block ids are read through the constant address space (scalar
  // loads, counted by lgkmcnt), each one segment ahead: a vector load of the
  // id would be waited for with vmcnt(0) before the segment's K / V loads
  // could issue, one dependent round trip per segment.
  typedef __attribute__((address_space(4))) const int32_t cint32;
  typedef __attribute__((address_space(4))) const float cfloat;
  const cint32* ids_l = (const cint32*)(p.ids + static_cast<int64_t>(layer) * p.ids_ls);
  auto id_at = [&](int s) { return s < p.n_hist ? ids_l[s] : 0; };
  // One segment of this wavefront (blk: its block id, for history segments).
  // int8 history segments (always the first n_hist segments) and bf16
  // segments are two instantiations of the body, run by two loops in segment
  // order, so neither carries the other's registers.
  auto segment = [&](const int sidx, const int blk, auto int8_tag, auto first_tag) __attribute__((always_inline)) {
    constexpr bool int8_seg = decltype(int8_tag)::value;
    constexpr bool first = decltype(first_tag)::value;
    const Seg g = make_seg_blk<FMT>(p, layer, h, sidx, blk);
    // an id outside the history attends nothing: no loads (a fully masked
    // segment would leave m, l and acc exactly as they are)
    if (g.type == kSegHist && g.vlen == 0) return;
    const int last = g.len - 1;

    // ---- K loads, S^T = K . Q^T on the matrix cores, V loads ----------------
    // K: lane (lg, ln) loads dims [32 s + 8 lg, +8) of key 16 i + ln (the
    // MFMA A operand); V: lane (lg, ln) loads dims [8 ln, +8) of key 4 j + lg.
    // With 4 query rows V is issued together with K, so a segment's 32 KiB
    // are in flight at once (the registers fit 2 waves per SIMD); wider
    // accumulators issue V after the MFMAs so K and V are not live together.
    constexpr bool kVEarly = (M == 4);
    // 4 query rows: one query group per (layer, KV head), so every selected
    // block is read once per launch -> history streamed past the caches
    // (non-temporal).  Under int8 history the bf16 sink / recent / chunk
    // segments, which the next step reads again, keep the default policy
    // (36-layer int8 32K step +3%); bf16 history streams them too (the
    // default policy there: no gain at 8K / 32K, slower at 128K).  Under
    // int8 history this body's bf16 instantiation sees no history segment,
    // so the choice is a compile-time one.
    constexpr bool kStream = (M == 4);
    constexpr bool nt_seg = kStream && (FMT == NKV_KV_BF16 || int8_seg);
    f32x4 c[4];
    uint4 va[16];
    // int8 history: the block's V scale (per-channel form, one scalar load)
    // or the fp16 K and V scales of this lane's keys 16 i + 4 lg .. + 3
    // (per-token form, 8-byte loads), issued with K and V
    float vs_blk = 1.0f;
    uint2 kts[4], vts[4];
    auto load_v = [&]() __attribute__((always_inline)) {
      if (int8_seg && kMfmaPV) {
        // 16 codes a lane: key 8 j + (lane >> 3), dims [16 (lane & 7), +16)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          va[j] = kv_load16<kStream>(g.vbase + min(8 * j + (lane >> 3), last) * g.rowb + (lane & 7) * 16);
      } else if (int8_seg) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint2 r = kv_load8<kStream>(g.vbase + min(4 * j + lg, last) * g.rowb + ln * 8);
          va[j] = make_uint4(r.x, r.y, 0u, 0u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j)
          va[j] = kv_load16<nt_seg>(g.vbase + min(4 * j + lg, last) * g.rowb + ln * 16);
      }
    };
    if (int8_seg) {
      uint4 kb[4][2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const char* rp = g.kbase + min(i * 16 + ln, last) * g.rowb + lg * 16;
        kb[i][0] = kv_load16<kStream>(rp);
        kb[i][1] = kv_load16<kStream>(rp + 64);
      }
      if (kVEarly) load_v();
      if (FMT == NKV_KV_INT8_CHANNEL)
        vs_blk = ((const cfloat*)p.v_scale)[(static_cast<int64_t>(layer) * p.hkv + h) * p.cap + g.blk];
      if (FMT == NKV_KV_INT8_TOKEN) {
        const int64_t tb = ((static_cast<int64_t>(layer) * p.hkv + h) * p.cap + g.blk) * kBlock + 4 * lg;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kts[i] = *reinterpret_cast<const uint2*>(p.k_tscale + tb + 16 * i);
          vts[i] = *reinterpret_cast<const uint2*>(p.v_tscale + tb + 16 * i);
        }
      }
      // every load of the segment issues before the first wait (left to
      // itself the scheduler holds the V loads back until K has arrived: a
      // second round trip per segment; +0.2-0.8% on the int8 step).  Not in
      // the first segment, whose query and scale registers are still live
      // (pinned there, the stream form spills), nor for bf16 segments, whose
      // waves already wait on a full memory pipeline (no gain measured).
      if constexpr (!first) {
        if (kVEarly) __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (first) make_bqs();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint4 w = kb[i][s >> 1];
          const uint32_t lo = (s & 1) ? w.z : w.x;
          const uint32_t hi = (s & 1) ? w.w : w.y;
          c[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(i8x8_to_bf16x8(lo, hi)), bqs[s], c[i], 0, 0, 0);
        }
      }
    } else {
      uint4 ka[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const char* rp = g.kbase + min(i * 16 + ln, last) * g.rowb + lg * 16;
#pragma unroll
        for (int s = 0; s < 4; ++s) ka[i][s] = kv_load16<nt_seg>(rp + s * 64);
      }
      if (kVEarly) load_v();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
          c[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka[i][s]), bq[s], c[i], 0, 0, 0);
      }
    }
    if (!kVEarly) {
      // the scheduling barrier keeps these loads after the MFMAs
      __builtin_amdgcn_sched_barrier(0);
      load_v();
    }

    // ---- masking, scale, online softmax ------------------------------------
    // c[i][e]: key tk = 16 i + 4 lg + e, query row ln.
    const uint8_t* allow_row =
        (g.type == kSegHist && p.allowed != nullptr)
            ? p.allowed + p.allowed_ls * layer + static_cast<int64_t>(my_t) * p.n_hist
            : nullptr;
    const bool seg_allowed = allow_row == nullptr || allow_row[g.u] != 0;
    float x[4][4];
    float cmax = -INFINITY;
    // the segment kind is uniform: one branch per segment picks the element
    // loop (a kind test per element compiles to a branch per element)
    auto mask = [&](auto kind_tag) __attribute__((always_inline)) {
      constexpr int KIND = decltype(kind_tag)::value;   // 0 history / sink, 1 ring, 2 chunk
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tk = i * 16 + lg * 4 + e;
          float v = c[i][e];
          bool ok = row_ok && tk < g.vlen && seg_allowed;
          if constexpr (KIND == 1) {
            int lp = g.off + tk - ring_base;
            if (lp < 0) lp += p.R;
            ok = ok && static_cast<unsigned>(lp - p.rec_lo) < static_cast<unsigned>(p.rec_len);
          } else if constexpr (KIND == 2) {
            if constexpr (PACKED) {
              ok = ok && (g.off + tk) - p.causal_off <= my_t;
              if (ok && p.tok_mask != nullptr)
                ok = p.tok_mask[static_cast<int64_t>(my_t) * p.n_chunk + g.off + tk] == 0;
            } else {
              ok = ok && (g.off + tk) <= my_t;
            }
          }
          if (FMT == NKV_KV_INT8_TOKEN && int8_seg) {
            const uint32_t w = e < 2 ? kts[i].x : kts[i].y;
            v *= f16_bits_to_f32(static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu)));
          }
          v = ok ? v * p.scale_log2 : -INFINITY;
          x[i][e] = v;
          cmax = fmaxf(cmax, v);
        }
      }
    };
    if (!int8_seg && g.type == kSegRecent)
      mask(std::integral_constant<int, 1>{});
    else if (!int8_seg && g.type == kSegChunk)
      mask(std::integral_constant<int, 2>{});
    else
      mask(std::integral_constant<int, 0>{});
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
    const float m_new = fmaxf(m_run, cmax);
    const float alpha = (m_new == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tk = i * 16 + lg * 4 + e;
        const float pe = (x[i][e] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(x[i][e] - m_new);
        lsum += pe;
        float pv = pe * vs_blk;
        if (FMT == NKV_KV_INT8_TOKEN && int8_seg) {
          const uint32_t w = e < 2 ? vts[i].x : vts[i].y;
          pv *= f16_bits_to_f32(static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu)));
        }
        if (kMfmaPV)
          x[i][e] = pv;
        else
          my_p[tk * kPRow + ln] = pv;
      }
    }
    l_run = l_run * alpha + lsum;
    m_run = m_new;

    if constexpr (kMfmaPV) {
      // ---- O^T += V^T . P^T on the matrix cores -----------------------------
      // V (int8 widened to bf16 exactly) -> LDS; P^T from registers: key
      // 32 k2 + 4 lg + e is x[2 k2][e], key 32 k2 + 16 + 4 lg + e is
      // x[2 k2 + 1][e], the same order the transposing reads give V^T.  P
      // enters as bf16 hi + lo parts (about 16 significant bits), so P.V
      // keeps fp32 accuracy.
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) oacc[dt] *= alpha;
      if (int8_seg) {
        // key 8 j + (lane >> 3): bf16 chunks 2 c and 2 c + 1 (c = lane & 7)
        // at positions (2 c ^ 2 (key & 3)) and the next
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = 8 * j + (lane >> 3);
          char* dst = my_v + key * 256 + (((2 * (lane & 7)) ^ (2 * (key & 3))) << 4);
          *reinterpret_cast<uint4*>(dst) = i8x8_to_bf16x8(va[j].x, va[j].y);
          *reinterpret_cast<uint4*>(dst + 16) = i8x8_to_bf16x8(va[j].z, va[j].w);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) *reinterpret_cast<uint4*>(my_v + j * 1024 + vw) = va[j];
      }
      wave_lds_sync();
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const float v8[8] = {x[2 * k2][0], x[2 * k2][1], x[2 * k2][2], x[2 * k2][3],
                             x[2 * k2 + 1][0], x[2 * k2 + 1][1], x[2 * k2 + 1][2], x[2 * k2 + 1][3]};
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hw[i] = stage::pack_bf16(v8[2 * i], v8[2 * i + 1]);
          lw[i] = stage::pack_bf16(v8[2 * i] - __uint_as_float(hw[i] << 16),
                                   v8[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u));
        }
        const bf16x8 bp = as_bf16x8(make_uint4(hw[0], hw[1], hw[2], hw[3]));
        const bf16x8 bl = as_bf16x8(make_uint4(lw[0], lw[1], lw[2], lw[3]));
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const char* vp = my_v + vtr[dt & 3] + (dt >> 2) * 128 + k2 * 8192;
          const stage::i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((stage::lds_i16x4*)(vp));
          const stage::i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((stage::lds_i16x4*)(vp + 4096));
          const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp, oacc[dt], 0, 0, 0);
          oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, oacc[dt], 0, 0, 0);
        }
      }
      wave_lds_sync();   // the next segment overwrites the V tile
      return;
    }
    if (lane < kMaxRows) s_alpha[wave][lane] = alpha;
    wave_lds_sync();

    // ---- O += P . V (fp32) --------------------------------------------------
#pragma unroll
    for (int n = 0; n < M; ++n) {
      const float al = s_alpha[wave][n];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[n][e] *= al;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int tk = 4 * j + lg;
      float vf[8];
      if (int8_seg) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t w = (e < 4) ? va[j].x : va[j].y;
          vf[e] = static_cast<float>(static_cast<int8_t>((w >> ((e & 3) * 8)) & 0xffu));
        }
      } else {
        vf[0] = bf16_lo(va[j].x); vf[1] = bf16_hi(va[j].x); vf[2] = bf16_lo(va[j].y); vf[3] = bf16_hi(va[j].y);
        vf[4] = bf16_lo(va[j].z); vf[5] = bf16_hi(va[j].z); vf[6] = bf16_lo(va[j].w); vf[7] = bf16_hi(va[j].w);
      }
      const float* prow = my_p + tk * kPRow;
#pragma unroll
      for (int n4 = 0; n4 < M; n4 += 4) {
        const float4 pp = *reinterpret_cast<const float4*>(prow + n4);
        const float pn[4] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[n4 + u][e] = __builtin_fmaf(pn[u], vf[e], acc[n4 + u][e]);
      }
    }
    wave_lds_sync();
  };
  int sidx = s_begin;
  int i8_end = min(p.n_hist, s_end);
  int bf_begin = -1, bf_end = s_end;
  if constexpr (stream && FMT != NKV_KV_BF16) {
    // A stream-form run [s_begin, s_end) of the group's items, read as an
    // even interleaving of its int8 history segments (16 KiB each) and its
    // bf16 sink / recent / chunk segments (32 KiB): of the group's first x
    // items, floor(x nb / nseg) are bf16 (nb = nseg - n_hist), kept in order
    // within each kind.  Consecutive runs still partition both kinds, and
    // every wavefront carries about the same bytes (in segment order the
    // wavefronts at a group's end took only bf16 segments, twice the bytes).
    const int nb16 = p.nseg - p.n_hist;
    const int c0 = (s_begin * nb16) / p.nseg, c1 = (s_end * nb16) / p.nseg;
    sidx = s_begin - c0;
    i8_end = s_end - c1;
    bf_begin = p.n_hist + c0;
    bf_end = p.n_hist + c1;
  }
  int blk = id_at(sidx);
  if constexpr (FMT != NKV_KV_BF16) {
    if (sidx < i8_end) {
      const int nb = id_at(sidx + s_step);   // in flight while this segment is attended
      // (an id outside the history attends nothing and issues no loads: bqs
      // is then formed at once)
      if (blk >= 0 && blk < p.cap)
        segment(sidx, blk, std::true_type{}, std::true_type{});
      else
        make_bqs();
      blk = nb;
      sidx += s_step;
    }
    for (; sidx < i8_end; sidx += s_step) {
      const int nb = id_at(sidx + s_step);
      segment(sidx, blk, std::true_type{}, std::false_type{});
      blk = nb;
    }
    load_bq();
    if (bf_begin >= 0) sidx = bf_begin;
  }
  for (; sidx < bf_end; sidx += s_step) {
    const int nb = id_at(sidx + s_step);
    segment(sidx, blk, std::false_type{}, std::false_type{});
    blk = nb;
  }

  // ---- reduce the wave's state across lane groups --------------------------
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if constexpr (!kMfmaPV) {
#pragma unroll
    for (int n = 0; n < M; ++n)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[n][e] += __shfl_xor(acc[n][e], 16);
        acc[n][e] += __shfl_xor(acc[n][e], 32);
      }
  }

  if constexpr (kMfmaPV && stream) {
    // the wavefront's own partial record: m, l, acc of rows ln < rows
    if (ln < rows) {
      float* part = p.partial + (static_cast<int64_t>(rec) * p.prow + ln) * kPartStride;
      if (lg == 0) {
        part[0] = m_run;
        part[1] = l_run;
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[2 + 16 * dt + 4 * lg + i] = oacc[dt][i];
    }
    return;
  }

  // ---- merge the 4 wavefronts in LDS (reusing the p tiles) -----------------
  __syncthreads();
  float* s_m = s_lds;                              // [waves][16]
  float* s_l = s_m + kAttendWaves * kMaxRows;      // [waves][16]
  float* s_acc = s_l + kAttendWaves * kMaxRows;    // [waves][M][128]
  if (lane < kMaxRows) {
    s_m[wave * kMaxRows + lane] = m_run;
    s_l[wave * kMaxRows + lane] = l_run;
  }
  if constexpr (kMfmaPV) {
    if (ln < M) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_acc[(wave * M + ln) * kHeadDim + 16 * dt + 4 * lg + i] = oacc[dt][i];
    }
  } else if (lg == 0) {
#pragma unroll
    for (int n = 0; n < M; ++n)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[(wave * M + n) * kHeadDim + ln * 8 + e] = acc[n][e];
  }
  __syncthreads();

  const int64_t grp = (static_cast<int64_t>(layer) * p.hkv + h) * p.nqg + qg;
  for (int idx = threadIdx.x; idx < M * kHeadDim; idx += kAttendThreads) {
    const int n = idx / kHeadDim, d = idx % kHeadDim;
    if (n >= rows) continue;
    float mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttendWaves; ++w) mt = fmaxf(mt, s_m[w * kMaxRows + n]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttendWaves; ++w) {
      const float mw = s_m[w * kMaxRows + n];
      const float sw = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - mt);
      L += s_l[w * kMaxRows + n] * sw;
      A += s_acc[(w * M + n) * kHeadDim + d] * sw;
    }
    if (p.splits == 1) {
      const int t = q0 + n / p.G;
      const int hh = h * p.G + n % p.G;
      p.out[p.q_ls * layer + (static_cast<int64_t>(t) * hq + hh) * kHeadDim + d] = f32_to_bf16(A / L);
    } else {
      float* part = p.partial + ((grp * p.splits + s_begin / kAttendWaves) * p.prow + n) * kPartStride;
      part[2 + d] = A;
      if (d == 0) {
        part[0] = mt;
        part[1] = L;
      }
    }
  }
  };

  if constexpr (STREAM && kMfmaPV && !PACKED) {
    // Stream form: wpg wavefronts per group (group g = (layer Hkv + h) nqg +
    // qg); wavefront j of group g attends the group's segments
    // [j nseg / wpg, (j + 1) nseg / wpg) and writes record w = g wpg + j.
    // Every run lies in one group (one call of `group`, no loop over groups:
    // 204-207 VGPRs and no scalar spills, against 231-253 VGPRs and 32-47
    // spilled scalars for runs that may cross a group boundary).
    const int w = static_cast<int>(blockIdx.x) * kAttendWaves + wave;
    const int g = w / p.stream_wpg, j = w % p.stream_wpg;
    if (g >= p.nlayers * p.hkv * p.nqg) return;
    const int sb = j * p.nseg / p.stream_wpg, se = (j + 1) * p.nseg / p.stream_wpg;
    const int lh = g / p.nqg;
    group(lh / p.hkv, lh % p.hkv, g % p.nqg, sb, 1, se, j == 0, w);
  } else {
    // split form: wavefront w of split s attends segments w + 4 s,
    // w + 4 s + 4 splits, ...
    group(blockIdx.z / p.nqg, blockIdx.y, blockIdx.z % p.nqg, blockIdx.x * kAttendWaves + wave,
          p.splits * kAttendWaves, p.nseg, blockIdx.x == 0, -1);
  }
}

// The wide few-query kernel: up to 32 query rows (two 16-column MFMA tiles)
// per (layer, KV head, query group), for verify-sized chunks (6 tokens x 4
// heads = 24 rows), which the 16-row kernel would split into two groups that
// each read every selected block.  Same segments, masks, split partials and
// numerics as attend_kernel's 4-row form: Q.K^T and P.V on the matrix cores,
// P as bf16 hi + lo parts (fp32-accurate P.V), int8 widened exactly with the
// scales folded into the query operand / p.  Registers: K (64) and the
// accumulators (32 logits, 64 O^T) are live together, so V is loaded once
// the Q.K^T products have consumed K (V's latency overlaps the softmax), and
// the query operands are read from LDS per product instead of held.
template <int FMT>
__global__ __launch_bounds__(kAttendThreads, 2) void attend_wide_kernel(const AttendParams p) {
  constexpr int NCT = kWideRows / 16;   // MFMA column tiles
  constexpr bool kI8 = FMT != NKV_KV_BF16;
  constexpr int kQCopies = kI8 ? 2 : 1;
  // V tiles of the four waves (16 KiB each), reused for the cross-wave merge
  __shared__ __attribute__((aligned(16))) char s_v[kAttendWaves * kVTileBytes];
  // B operands: [copy][ct][s][lane] (copy 1, int8 history: the query over
  // the dims its 16-byte key loads put in MFMA step s,
  // [64 (s >> 1) + 16 lg + 8 (s & 1), +8),
  // K-scaled for per-channel scales); after the segment loop, the merge's m
  // and l
  __shared__ __attribute__((aligned(16))) bf16x8 s_q[kQCopies][NCT][4][kWave];
  static_assert(sizeof(s_q) >= 2 * kAttendWaves * kWideRows * sizeof(float), "m, l fit the operand area");
  float (*s_ml)[kAttendWaves][kWideRows] = reinterpret_cast<float (*)[kAttendWaves][kWideRows]>(&s_q[0][0][0][0]);

  // (group, split): the grid's coordinates, or the tiered plan's order --
  // the first wide_ga groups' wide_sa splits each, then the rest's wide_sb
  int split, ns, layer, h, qg;
  int64_t grp, rbase;
  if (p.wide_sa > 0) {
    const int bid = blockIdx.x;
    const int na = p.wide_ga * p.wide_sa;
    if (bid < na) {
      grp = bid / p.wide_sa;
      split = bid % p.wide_sa;
      ns = p.wide_sa;
      rbase = grp * p.wide_sa;
    } else {
      grp = p.wide_ga + (bid - na) / p.wide_sb;
      split = (bid - na) % p.wide_sb;
      ns = p.wide_sb;
      rbase = na + (grp - p.wide_ga) * p.wide_sb;
    }
    qg = static_cast<int>(grp % p.nqg);
    h = static_cast<int>((grp / p.nqg) % p.hkv);
    layer = static_cast<int>(grp / (static_cast<int64_t>(p.nqg) * p.hkv));
  } else {
    split = blockIdx.x;
    h = blockIdx.y;
    layer = blockIdx.z / p.nqg;
    qg = blockIdx.z % p.nqg;
    ns = p.splits;
    grp = (static_cast<int64_t>(layer) * p.hkv + h) * p.nqg + qg;
    rbase = grp * p.splits;
  }
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int ln = lane & 15;
  const int lg = lane >> 4;
  const int hq = p.hkv * p.G;
  const int q0 = qg * p.qpg;
  const int rows = min(p.qpg, p.tq - q0) * p.G;

  int write_slot = p.write_slot, ring_base = p.ring_base;
  if (p.ring_start != nullptr) {
    write_slot = static_cast<int>(static_cast<uint32_t>(p.ring_start[layer]) % static_cast<uint32_t>(p.R));
    ring_base = write_slot + 1 == p.R ? 0 : write_slot + 1;
  }
  if (p.zero_keys != nullptr && split == 0 && h == 0 && qg == 0) {
    uint32_t* zk = p.zero_keys + static_cast<int64_t>(layer) * p.zero_n;
    for (int i = threadIdx.x; i < p.zero_n; i += kAttendThreads) zk[i] = 0u;
  }
  if (write_slot >= 0 && split == 0 && qg == 0 && wave == 0 && lane < 32) {
    const int which = lane >> 4;
    const int c = lane & 15;
    const uint4* src = reinterpret_cast<const uint4*>(
        (which ? p.v_new : p.k_new) + p.kv_ls * layer + static_cast<int64_t>(h) * kHeadDim);
    uint4* dst = reinterpret_cast<uint4*>((which ? p.rec_v : p.rec_k) + p.rec_ls * layer +
                                         (static_cast<int64_t>(h) * p.R + write_slot) * kHeadDim);
    dst[c] = src[c];
  }

  // ---- query operands into LDS: wave w fills column tile ct = w & 1, dim
  // chunks s = 2 (w >> 1) + {0, 1} (row n = 16 ct + ln, dims 32 s + 8 lg) --
  {
    const int ct = wave & 1;
    const int n = 16 * ct + ln;
    const bool ok = n < rows;
    const int t = q0 + (ok ? n / p.G : 0);
    const int hh = h * p.G + n % p.G;
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      const int s = 2 * (wave >> 1) + si;
      const int d0 = s * 32 + lg * 8;
      const uint16_t* qrow = p.q + p.q_ls * layer + (static_cast<int64_t>(t) * hq + hh) * kHeadDim;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (ok) v = *reinterpret_cast<const uint4*>(qrow + d0);
      s_q[0][ct][s][lane] = as_bf16x8(v);
      if constexpr (kI8) {
        const int dp = (s >> 1) * 64 + lg * 16 + (s & 1) * 8;
        uint4 vp = make_uint4(0u, 0u, 0u, 0u);
        if (ok) vp = *reinterpret_cast<const uint4*>(qrow + dp);
        if constexpr (FMT == NKV_KV_INT8_CHANNEL) {
          const float* ks = p.k_scale + static_cast<int64_t>(layer) * p.hkv * kHeadDim + h * kHeadDim + dp;
          const uint32_t w[4] = {vp.x, vp.y, vp.z, vp.w};
          uint32_t o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float a = bf16_lo(w[i]) * ks[2 * i];
            const float b = bf16_hi(w[i]) * ks[2 * i + 1];
            o[i] = static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
          }
          vp = make_uint4(o[0], o[1], o[2], o[3]);
        }
        s_q[1][ct][s][lane] = as_bf16x8(vp);
      }
    }
  }
  __syncthreads();

  // per column tile: row n = 16 ct + ln
  bool row_ok[NCT];
  int my_t[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int n = 16 * ct + ln;
    row_ok[ct] = n < rows;
    my_t[ct] = q0 + (row_ok[ct] ? n / p.G : 0);
  }
  float m_run[NCT], l_run[NCT];
  f32x4 oacc[8][NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    m_run[ct] = -INFINITY;
    l_run[ct] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[dt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  char* my_v = s_v + wave * kVTileBytes;
  const int vw = lg * 256 + ((ln ^ (2 * lg)) << 4);
  int vtr[4];
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4)
    vtr[q4] = (4 * lg + (ln >> 2)) * 256 + ((2 * (q4 ^ (ln >> 2)) + ((ln & 3) >> 1)) << 4) + 8 * (ln & 1);
  const int nwaves = ns * kAttendWaves;

  // A history segment whose id lies outside the history attends nothing (a
  // fully masked segment would leave m, l and acc as they are): passed over.
  // The ids are read through the constant address space (scalar loads,
  // counted by lgkmcnt): a vector load would be waited for with vmcnt(0),
  // draining the current segment's loads with it.
  typedef __attribute__((address_space(4))) const int32_t cint32;
  typedef __attribute__((address_space(4))) const float cfloat;
  const cint32* ids_l = (const cint32*)(p.ids + static_cast<int64_t>(layer) * p.ids_ls);
  auto skip_empty = [&](int sidx, int end) {
    while (sidx < end && sidx < p.n_hist) {
      const int blk = ids_l[sidx];
      if (blk >= 0 && blk < p.cap) break;
      sidx += nwaves;
    }
    return sidx;
  };

  // The wave's segments sidx, sidx + nwaves, ... below `end`, all int8
  // history (int8 tag) or all bf16.  Returns the first index at or past end.
  // Two forms, chosen by measurement on the 36-layer 16K verify round:
  //   registers (bf16 history, int8 history): bf16 K, then V once Q.K^T has
  //   consumed K (the registers hold one of them; 374 vs 387 us); int8 K and
  //   V (8 bytes a lane and row) together.  V is written to the LDS tile
  //   (int8 widened exactly on the way).
  //   direct copies (the bf16 sink / recent / chunk segments of int8
  //   history): V goes global -> LDS without registers, issued with K, and
  //   the next segment's K loads go out once Q.K^T is done (per-token int8
  //   324 vs 338 us).
  // With one query group per (layer, KV head) (verify's draft tokens) each
  // history block is read once per launch: its loads are non-temporal, while
  // the sink / recent / chunk segments keep the default policy (the 36-layer
  // 16K verify round -4% bf16, -3% int8; all segments non-temporal -2%).
  const bool nt_hist = p.nqg == 1;
  auto run_phase = [&](int sidx, int end, auto int8_tag) __attribute__((always_inline)) {
    constexpr bool int8_seg = decltype(int8_tag)::value;
    constexpr bool reg_v = int8_seg || FMT == NKV_KV_BF16;
    // the next segment's K loaded once Q.K^T is done (the copy form, whose V
    // holds no registers; measured no gain for int8 history's register form)
    constexpr bool prefetch_k = !reg_v;
    const int qsel = int8_seg ? 1 : 0;
    // bf16 keys: dims [32 s + 8 lg, +8) of key 16 i + ln in ka[i][s]; int8
    // keys: dims [16 lg, +16) and [64 + 16 lg, +16) in ka[i][0..1] (16-byte loads)
    uint4 ka[4][4];
    // (int8 segments choose the policy by one uniform branch around their
    // loads -- a policy selected per load compiles to a branch per load:
    // int8 verify round -2.7%; the bf16 segments keep the per-load choice,
    // which measured faster for them)
    auto load_k = [&](const Seg& g) __attribute__((always_inline)) {
      const int last = g.len - 1;
      if constexpr (int8_seg) {
        auto ld = [&](auto nt_tag) __attribute__((always_inline)) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const char* rp = g.kbase + min(i * 16 + ln, last) * g.rowb + lg * 16;
            ka[i][0] = kv_load16<decltype(nt_tag)::value>(rp);
            ka[i][1] = kv_load16<decltype(nt_tag)::value>(rp + 64);
          }
        };
        if (nt_hist)
          ld(std::true_type{});
        else
          ld(std::false_type{});
      } else {
        // (under int8 history the bf16 segments are never history blocks)
        const bool nt = FMT == NKV_KV_BF16 && nt_hist && g.type == kSegHist;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const char* rp = g.kbase + min(i * 16 + ln, last) * g.rowb + lg * 16;
#pragma unroll
          for (int s = 0; s < 4; ++s) ka[i][s] = nt ? kv_load16<true>(rp + s * 64) : kv_load16<false>(rp + s * 64);
        }
      }
    };
    // bf16 V of segment g -> this wave's V tile: copy j puts key 4 j + lg,
    // chunk ln' ^ 2 lg at lane ln' of its 1 KiB, i.e. chunk c of key k at
    // j * 1024 + lg * 256 + ((c ^ 2 lg) << 4), the layout the transposing
    // reads expect; rows past the segment read as zero (bounded descriptor)
    auto copy_v = [&](const Seg& g) __attribute__((always_inline)) {
      const stage::rsrc_words rv = stage::rsrc_of(g.vbase, static_cast<uint32_t>(g.len * g.rowb));
#pragma unroll
      for (int j = 0; j < 16; ++j)
        stage::lds_copy16(rv, my_v + j * 1024, (4 * j + lg) * g.rowb + ((ln ^ (2 * lg)) << 4));
    };
    sidx = skip_empty(sidx, end);
    if (sidx >= end) return sidx;
    Seg g = make_seg<FMT>(p, layer, h, sidx);
    if constexpr (prefetch_k) load_k(g);
    if constexpr (!reg_v) copy_v(g);
    while (true) {
      const int last = g.len - 1;
      if constexpr (!prefetch_k) load_k(g);
      // int8 history: V (8 bytes a lane and key row, 32 registers) goes out
      // with K, so the segment's 16 KiB are in flight together, and so do the
      // block's V scale (per-channel form, a scalar load) or the fp16 K and V
      // scales of this lane's keys 16 i + 4 lg .. + 3 (per-token form)
      // (int8 V: 16 codes a lane, key 8 j + (lane >> 3), dims [16 (lane & 7), +16))
      uint4 va8[int8_seg ? 8 : 1];
      float vs_blk = 1.0f;
      uint2 kts[4], vts[4];
      if constexpr (int8_seg) {
        auto ld = [&](auto nt_tag) __attribute__((always_inline)) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            va8[j] = kv_load16<decltype(nt_tag)::value>(g.vbase + min(8 * j + (lane >> 3), last) * g.rowb +
                                                        (lane & 7) * 16);
        };
        if (nt_hist)
          ld(std::true_type{});
        else
          ld(std::false_type{});
        if (FMT == NKV_KV_INT8_CHANNEL)
          vs_blk = ((const cfloat*)p.v_scale)[(static_cast<int64_t>(layer) * p.hkv + h) * p.cap + g.blk];
        if (FMT == NKV_KV_INT8_TOKEN) {
          const int64_t tb = ((static_cast<int64_t>(layer) * p.hkv + h) * p.cap + g.blk) * kBlock + 4 * lg;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            kts[i] = *reinterpret_cast<const uint2*>(p.k_tscale + tb + 16 * i);
            vts[i] = *reinterpret_cast<const uint2*>(p.v_tscale + tb + 16 * i);
          }
        }
      }
      // per-query history flags of this segment (verify's union), loaded
      // before the products so their wait is the loads' own
      int hidden[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        hidden[ct] = 0;
        if (g.type == kSegHist && p.allowed != nullptr)
          hidden[ct] = p.allowed[p.allowed_ls * layer + static_cast<int64_t>(my_t[ct]) * p.n_hist + g.u] == 0;
      }
      // the next segment (its id is a scalar load, in flight with K)
      const int snext = skip_empty(sidx + nwaves, end);
      const bool more = snext < end;
      Seg gn = g;
      if (more) gn = make_seg<FMT>(p, layer, h, snext);
      // ---- S^T = K . Q^T on the matrix cores ---------------------------------
      f32x4 c[4][NCT];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) c[i][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        bf16x8 bq[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) bq[ct] = s_q[qsel][ct][s][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16x8 a;
          if constexpr (int8_seg) {
            const uint4 w = ka[i][s >> 1];
            a = as_bf16x8(i8x8_to_bf16x8((s & 1) ? w.z : w.x, (s & 1) ? w.w : w.y));
          } else
            a = as_bf16x8(ka[i][s]);
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) c[i][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[ct], c[i][ct], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // register form, bf16: V after the products (lane (lg, ln): dims
      // [8 ln, +8) of key 4 j + lg)
      uint4 va[reg_v && !int8_seg ? 16 : 1];
      if constexpr (reg_v && !int8_seg) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
          va[j] = nt_hist && g.type == kSegHist
                      ? kv_load16<true>(g.vbase + min(4 * j + lg, last) * g.rowb + ln * 16)
                      : kv_load16<false>(g.vbase + min(4 * j + lg, last) * g.rowb + ln * 16);
      }
      // the next segment's K, issued after this segment's V
      if constexpr (prefetch_k) {
        if (more) load_k(gn);
      }
      __builtin_amdgcn_sched_barrier(0);

      // ---- masking, scale, online softmax per column tile ------------------
      // c[i][ct][e]: key 16 i + 4 lg + e, row 16 ct + ln
      // Visibility, branch-free: key tk of the segment is visible to column
      // tile ct iff d = 4 lg + (16 i + e) - thr[ct] <= 0, where thr[ct] is the
      // last visible key (-1: none; the row's validity, the per-query history
      // flags and the chunk's causal edge folded in); a ring piece also needs
      // the slot's logical position in the window: x(tk) - (rec_len - 1) <= 0.
      int base[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        int thr = g.vlen - 1;
        if (g.type == kSegChunk) thr = min(thr, my_t[ct] - g.off);
        if (hidden[ct]) thr = -1;
        if (!row_ok[ct]) thr = -1;
        base[ct] = 4 * lg - thr;
      }
      // ring piece: x = (slot - ring_base - rec_lo) mod R for slot off + key
      int ra = 0;
      const bool ring = g.type == kSegRecent;
      if (ring) {
        ra = (g.off - ring_base - p.rec_lo) % p.R;
        ra = ra < 0 ? ra + p.R : ra;
      }
      // fp16 scale of key 16 i + 4 lg + e from a lane's 8-byte load
      auto tscale = [](const uint2 (&w)[4], int i, int e) {
        const uint32_t x = e < 2 ? w[i].x : w[i].y;
        return f16_bits_to_f32(static_cast<uint16_t>((e & 1) ? (x >> 16) : (x & 0xffffu)));
      };
      float alpha[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        float cmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            bool ok = base[ct] + (16 * i + e) <= 0;
            if (ring) {
              int x = ra + 16 * i + 4 * lg + e;
              x -= p.R & ((p.R - 1 - x) >> 31);
              ok = ok && x < p.rec_len;
            }
            float v = c[i][ct][e];
            if constexpr (FMT == NKV_KV_INT8_TOKEN && int8_seg) v *= tscale(kts, i, e);
            v = ok ? v * p.scale_log2 : -INFINITY;
            c[i][ct][e] = v;
            cmax = fmaxf(cmax, v);
          }
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float m_new = fmaxf(m_run[ct], cmax);
        alpha[ct] = (m_new == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m_run[ct] - m_new);
        float lsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = c[i][ct][e];
            const float pe = (x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(x - m_new);
            lsum += pe;
            float pv = pe * vs_blk;
            if (FMT == NKV_KV_INT8_TOKEN && int8_seg) pv *= tscale(vts, i, e);
            c[i][ct][e] = pv;
          }
        }
        l_run[ct] = l_run[ct] * alpha[ct] + lsum;
        m_run[ct] = m_new;
      }

      // ---- V in the LDS tile, O^T += V^T . P^T -------------------------------
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) oacc[dt][ct] *= alpha[ct];
      if constexpr (reg_v && int8_seg) {
        // key 8 j + (lane >> 3): bf16 chunks 2 c and 2 c + 1 (c = lane & 7)
        // at positions (2 c ^ 2 (key & 3)) and the next
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = 8 * j + (lane >> 3);
          char* dst = my_v + key * 256 + (((2 * (lane & 7)) ^ (2 * (key & 3))) << 4);
          *reinterpret_cast<uint4*>(dst) = i8x8_to_bf16x8(va8[j].x, va8[j].y);
          *reinterpret_cast<uint4*>(dst + 16) = i8x8_to_bf16x8(va8[j].z, va8[j].w);
        }
        wave_lds_sync();
      } else if constexpr (reg_v) {
#pragma unroll
        for (int j = 0; j < 16; ++j) *reinterpret_cast<uint4*>(my_v + j * 1024 + vw) = va[j];
        wave_lds_sync();
      } else {
        // the V copies have landed: they were issued before the next K loads
        // (16 loads), which may stay in flight
        if (more)
          __builtin_amdgcn_s_waitcnt(0x4F70);   // vmcnt(16)
        else
          __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        __builtin_amdgcn_wave_barrier();
      }
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        bf16x8 bp[NCT], bl[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          const float v8[8] = {c[2 * k2][ct][0], c[2 * k2][ct][1], c[2 * k2][ct][2], c[2 * k2][ct][3],
                               c[2 * k2 + 1][ct][0], c[2 * k2 + 1][ct][1], c[2 * k2 + 1][ct][2], c[2 * k2 + 1][ct][3]};
          uint32_t hw[4], lw[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            hw[i] = stage::pack_bf16(v8[2 * i], v8[2 * i + 1]);
            lw[i] = stage::pack_bf16(v8[2 * i] - __uint_as_float(hw[i] << 16),
                                     v8[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u));
          }
          bp[ct] = as_bf16x8(make_uint4(hw[0], hw[1], hw[2], hw[3]));
          bl[ct] = as_bf16x8(make_uint4(lw[0], lw[1], lw[2], lw[3]));
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const char* vp = my_v + vtr[dt & 3] + (dt >> 2) * 128 + k2 * 8192;
          const stage::i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((stage::lds_i16x4*)(vp));
          const stage::i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((stage::lds_i16x4*)(vp + 4096));
          const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            oacc[dt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[ct], oacc[dt][ct], 0, 0, 0);
            oacc[dt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[ct], oacc[dt][ct], 0, 0, 0);
          }
        }
      }
      wave_lds_sync();   // every read of the V tile is done before it is refilled
      if (!more) return snext;
      sidx = snext;
      g = gn;
      if constexpr (!reg_v) copy_v(g);
    }
  };
  int sidx = split * kAttendWaves + wave;
  if constexpr (kI8) sidx = run_phase(sidx, p.n_hist, std::true_type{});
  run_phase(sidx, p.nseg, std::false_type{});

  // ---- merge the 4 wavefronts in LDS (reusing the V tiles) -----------------
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    l_run[ct] += __shfl_xor(l_run[ct], 16);
    l_run[ct] += __shfl_xor(l_run[ct], 32);
  }
  __syncthreads();   // every wave is done with its V tile and the query operands
  float* s_acc = reinterpret_cast<float*>(s_v);   // [waves][32][128]
  if (lg == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      s_ml[0][wave][16 * ct + ln] = m_run[ct];
      s_ml[1][wave][16 * ct + ln] = l_run[ct];
    }
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<f32x4*>(s_acc + ((wave * kWideRows + 16 * ct + ln) * kHeadDim) + 16 * dt + 4 * lg) =
          oacc[dt][ct];
  __syncthreads();

  for (int idx = threadIdx.x; idx < kWideRows * kHeadDim; idx += kAttendThreads) {
    const int n = idx / kHeadDim, d = idx % kHeadDim;
    if (n >= rows) continue;
    float mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttendWaves; ++w) mt = fmaxf(mt, s_ml[0][w][n]);
    float L = 0.0f, A = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttendWaves; ++w) {
      const float mw = s_ml[0][w][n];
      const float sw = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - mt);
      L += s_ml[1][w][n] * sw;
      A += s_acc[(w * kWideRows + n) * kHeadDim + d] * sw;
    }
    if (p.splits == 1) {
      const int t = q0 + n / p.G;
      const int hh = h * p.G + n % p.G;
      p.out[p.q_ls * layer + (static_cast<int64_t>(t) * hq + hh) * kHeadDim + d] = f32_to_bf16(A / L);
    } else {
      float* part = p.partial + ((rbase + split) * p.prow + n) * kPartStride;
      part[2 + d] = A;
      if (d == 0) {
        part[0] = mt;
        part[1] = L;
      }
    }
  }
}

// Merge the split partials: one workgroup per (KV head, layer x group, 4
// rows), 64 threads per row with 2 output dims each.  Every load of a
// thread (each split's m, l and its two acc values) is issued before the
// first is used, so the merge is one memory round trip.  Runs after the
// attention on the same stream, so the partials are visible without
// device-scope fences.
constexpr int kMergeRows = 4;
constexpr int kMergeThreads = kMergeRows * 64;
__global__ __launch_bounds__(kMergeThreads) void attend_merge_kernel(const AttendParams p) {
  const int h = blockIdx.x;
  const int layer = blockIdx.y / p.nqg;
  const int qg = blockIdx.y % p.nqg;
  const int n = blockIdx.z * kMergeRows + (threadIdx.x >> 6);
  const int d0 = (threadIdx.x & 63) * 2;
  const int hq = p.hkv * p.G;
  const int q0 = qg * p.qpg;
  const int rows = min(p.qpg, p.tq - q0) * p.G;
  // device-ring decode: the attention has read this layer's ring start, so
  // one thread of the layer's first merge workgroup moves it one slot
  if (p.ring_start != nullptr && h == 0 && qg == 0 && blockIdx.z == 0 && threadIdx.x == 0) {
    int32_t* rs = const_cast<int32_t*>(p.ring_start) + layer;
    const int v = static_cast<int>(static_cast<uint32_t>(*rs) % static_cast<uint32_t>(p.R));
    *rs = v + 1 == p.R ? 0 : v + 1;
  }
  if (n >= rows) return;
  const int64_t grp = (static_cast<int64_t>(layer) * p.hkv + h) * p.nqg + qg;
  // split form: records grp * splits .. + splits - 1; stream form: the
  // group's wavefronts' records grp * wpg .. + wpg - 1
  int64_t first = grp * p.splits;
  int nrec = p.splits;
  if (p.wide_sa > 0) {   // the wide kernel's tiered plan
    const int64_t na = static_cast<int64_t>(p.wide_ga) * p.wide_sa;
    first = grp < p.wide_ga ? grp * p.wide_sa : na + (grp - p.wide_ga) * p.wide_sb;
    nrec = grp < p.wide_ga ? p.wide_sa : p.wide_sb;
  }
  if (p.stream_wpg > 0) {
    first = grp * p.stream_wpg;
    nrec = p.stream_wpg;
  }
  const float* base = p.partial + (first * p.prow + n) * kPartStride;
  const int64_t sstride = static_cast<int64_t>(p.prow) * kPartStride;
  float L = 0.0f, A0 = 0.0f, A1 = 0.0f;
  // up to 8 records at a time: all their loads in flight together
  float mt = -INFINITY;
  for (int s0 = 0; s0 < nrec; s0 += 8) {
    float m[8], l[8];
    float2 a[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = min(s0 + i, nrec - 1);
      const float* ps = base + s * sstride;
      m[i] = ps[0];
      l[i] = ps[1];
      // the record is [m, l, acc[128]] at an even float offset: 8-byte loads
      a[i] = *reinterpret_cast<const float2*>(ps + 2 + d0);
    }
    float mb = mt;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (s0 + i < nrec) mb = fmaxf(mb, m[i]);
    // rescale what the earlier batches summed to the new reference max
    const float r = (mt == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mt - mb);
    L *= r;
    A0 *= r;
    A1 *= r;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (s0 + i >= nrec) break;
      const float sw = (m[i] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m[i] - mb);
      L += l[i] * sw;
      A0 += a[i].x * sw;
      A1 += a[i].y * sw;
    }
    mt = mb;
  }
  const int t = q0 + n / p.G;
  const int hh = h * p.G + n % p.G;
  *reinterpret_cast<uint32_t*>(p.out + p.q_ls * layer + (static_cast<int64_t>(t) * hq + hh) * kHeadDim + d0) =
      static_cast<uint32_t>(f32_to_bf16(A0 / L)) | (static_cast<uint32_t>(f32_to_bf16(A1 / L)) << 16);
}

// Device-ring decode: every layer's ring start moves one slot (mod R) once
// the step's attention has read it; the next launch on the stream sees it.
__global__ __launch_bounds__(kWave) void ring_advance_kernel(int32_t* ring_start, int n, int R) {
  const int i = blockIdx.x * kWave + threadIdx.x;
  if (i < n) {
    const int v = static_cast<int>(static_cast<uint32_t>(ring_start[i]) % static_cast<uint32_t>(R));
    ring_start[i] = v + 1 == R ? 0 : v + 1;
  }
}

template <int FMT, bool PACKED = false>
int launch_fmt(int M, dim3 grid, hipStream_t s, const AttendParams& p) {
  if (p.stream_wpg > 0) {
    if (M != 4 || PACKED) return -1;
    hipLaunchKernelGGL((attend_kernel<FMT, 4, false, true>), grid, dim3(kAttendThreads), 0, s, p);
    return 0;
  }
  switch (M) {
    case 4: hipLaunchKernelGGL((attend_kernel<FMT, 4, PACKED>), grid, dim3(kAttendThreads), 0, s, p); return 0;
    case 8: hipLaunchKernelGGL((attend_kernel<FMT, 8, PACKED>), grid, dim3(kAttendThreads), 0, s, p); return 0;
    case 16: hipLaunchKernelGGL((attend_kernel<FMT, 16, PACKED>), grid, dim3(kAttendThreads), 0, s, p); return 0;
    case kWideRows:
      if (PACKED) return -1;
      hipLaunchKernelGGL((attend_wide_kernel<FMT>), grid, dim3(kAttendThreads), 0, s, p);
      return 0;
    default: return -1;
  }
}

// Query rows per group and the kernel's row count for a given (tq, G): one
// 16-row MFMA tile when the chunk's rows fit it, else groups of two tiles
// (the wide kernel).
void group_shape(int tq, int G, int* qpg, int* M) {
  if (tq * G > kMaxRows) {
    int per = kWideRows / G;
    if (per > tq) per = tq;
    *qpg = per;
    *M = kWideRows;
    return;
  }
  int per = kMaxRows / G;          // queries that fit one MFMA tile
  if (per > tq) per = tq;
  *qpg = per;
  const int rows = per * G;
  *M = rows <= 4 ? 4 : (rows <= 8 ? 8 : 16);
}

}  // namespace

// The few-query kernel over (split, KV head, layer x query group), then the
// split merge.
// Timing marks of the calling host thread (nkv_set_attend_marks): recorded on
// the launch stream right before and right after the attention kernel (before
// its split merge); null: none.
thread_local hipEvent_t g_mark_before = nullptr;
thread_local hipEvent_t g_mark_after = nullptr;

int record_mark(hipEvent_t e, hipStream_t s) {
  if (e == nullptr) return NKV_OK;
  const hipError_t err = hipEventRecord(e, s);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    set_error("nkv_attend: recording a timing mark failed (%s)", hipGetErrorString(err));
    return NKV_ERR_HIP;
  }
  return NKV_OK;
}

int launch_grouped(int hkv, int kv_format, int num_layers, int tq, AttendParams& p, hipStream_t s) {
  int qpg, M;
  group_shape(tq, p.G, &qpg, &M);
  p.qpg = qpg;
  p.nqg = (tq + qpg - 1) / qpg;
  p.prow = M > kMaxRows ? kWideRows : kMaxRows;
  dim3 grid(p.splits, hkv, num_layers * p.nqg);
  int bad = 0;
  const bool packed = p.tok_mask != nullptr || p.causal_off != 0;
  NKV_CHECK_SUPPORTED(!packed || kv_format == NKV_KV_BF16, "nkv_attend: caller-packed keys must be bf16");
  if (p.splits == 0 && M == kWideRows && !packed) {
    // the wide kernel's tiered plan: its workgroups (two per CU) fill two
    // rounds of the device, the first with pieces of the first groups'
    // segment lists, the second with pieces about 3/4 their size of the
    // rest's, which also back-fill the slots the first round's slower
    // workgroups free late.  The uniform split form's last round runs partly
    // empty and latency-bound: 36-layer 16K verify round, 6 tokens, us at the
    // uniform 3 splits vs this plan (3 / 4 splits) vs 2 / 16: bf16 330 / 327 /
    // 328, int8 267 / 256 / 268, per-token int8 271 / 260 / 269.
    const int cus = device_cus();
    const int64_t slots = std::min<int64_t>(cus > 0 ? 2 * static_cast<int64_t>(cus) : kWidePlanSlotsMax,
                                            kWidePlanSlotsMax);
    const int64_t groups = static_cast<int64_t>(num_layers) * hkv * p.nqg;
    // a piece keeps at least two segments per wavefront
    const int smax = std::max(1, std::min(64, p.nseg / (2 * kAttendWaves)));
    int sa = 1, sb = 1;
    int64_t ga = groups;
    if (groups < slots) {
      // ga sa = slots and (groups - ga) sb = slots with sb = 4/3 sa give
      // sa = 7 slots / (4 groups)
      sa = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((7 * slots + 2 * groups) / (4 * groups), smax)));
      ga = std::min<int64_t>(groups, slots / sa);
      const int64_t gb = groups - ga;
      sb = gb > 0 ? static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(slots / gb, smax))) : 1;
    }
    p.wide_ga = static_cast<int>(ga);
    p.wide_sa = sa;
    p.wide_sb = sb;
    grid = dim3(static_cast<unsigned>(ga * sa + (groups - ga) * sb), 1, 1);
  } else if (p.splits == 0) {
    // stream form: one resident round of wavefronts (two workgroups per CU),
    // the same number per group, sharing each group's segments evenly
    NKV_CHECK_SUPPORTED(M == 4 && !packed,
                        "nkv_attend: the stream form (splits 0) takes groups of at most 4 query rows and no "
                        "caller-packed keys (got %d rows%s)", qpg * p.G, packed ? ", packed keys" : "");
    const int cus = device_cus();
    const int64_t waves = cus > 0 ? std::min<int64_t>(static_cast<int64_t>(cus) * 4 * NKV_ATTEND_DECODE_WAVES,
                                                      kStreamWavesMax)
                                  : kStreamWavesMax;
    const int64_t groups = static_cast<int64_t>(num_layers) * hkv * p.nqg;
    const int64_t wpg = std::max<int64_t>(1, std::min<int64_t>(waves / groups, p.nseg));
    NKV_CHECK_SUPPORTED(groups * wpg < (int64_t{1} << 31),
                        "nkv_attend: %lld groups are too many for the stream form", static_cast<long long>(groups));
    p.stream_wpg = static_cast<int>(wpg);
    p.prow = kStreamRows;
    grid = dim3(static_cast<unsigned>((groups * wpg + kAttendWaves - 1) / kAttendWaves), 1, 1);
  }
  if (const int rc = record_mark(g_mark_before, s); rc != NKV_OK) return rc;
  switch (kv_format) {
    case NKV_KV_BF16:
      bad = packed ? launch_fmt<NKV_KV_BF16, true>(M, grid, s, p) : launch_fmt<NKV_KV_BF16>(M, grid, s, p);
      break;
    case NKV_KV_INT8_CHANNEL: bad = launch_fmt<NKV_KV_INT8_CHANNEL>(M, grid, s, p); break;
    case NKV_KV_INT8_TOKEN: bad = launch_fmt<NKV_KV_INT8_TOKEN>(M, grid, s, p); break;
    default: bad = -1;
  }
  NKV_CHECK_SUPPORTED(bad == 0, "nkv_attend: unsupported row count %d / kv_format %d", M, kv_format);
  if (const int rc = record_mark(g_mark_after, s); rc != NKV_OK) return rc;
  if (p.splits != 1)
    hipLaunchKernelGGL(attend_merge_kernel, dim3(hkv, num_layers * p.nqg, (qpg * p.G + kMergeRows - 1) / kMergeRows),
                       dim3(kMergeThreads), 0, s, p);
  return NKV_OK;
}

}  // namespace nkv

using namespace nkv;

extern "C" int nkv_set_attend_marks(void* before, void* after) {
  g_mark_before = static_cast<hipEvent_t>(before);
  g_mark_after = static_cast<hipEvent_t>(after);
  return NKV_OK;
}

extern "C" int64_t nkv_attend_workspace_floats(int num_layers, int num_kv_heads, int num_heads,
                                               int tq, int splits) {
  if (num_layers < 1 || num_kv_heads < 1 || num_heads < num_kv_heads || tq < 1 || splits < 0) return 0;
  int qpg, M;
  group_shape(tq, num_heads / num_kv_heads, &qpg, &M);
  const int64_t nqg = (tq + qpg - 1) / qpg;
  if (splits == 0) {
    const int64_t groups = static_cast<int64_t>(num_layers) * num_kv_heads * nqg;
    // the wide kernel's tiered plan: at most two rounds of resident
    // workgroups' records (or one per group when the groups fill a round)
    if (M == kWideRows) return std::max<int64_t>(2 * kWidePlanSlotsMax, groups) * kWideRows * kPartStride;
    // stream form: one record per wavefront, groups x wpg <= max(groups,
    // kStreamWavesMax) of them
    if (M != 4) return 0;
    return (kStreamWavesMax + groups) * kStreamRows * kPartStride;
  }
  const int prow = M > kMaxRows ? kWideRows : kMaxRows;
  return static_cast<int64_t>(num_layers) * num_kv_heads * nqg * splits * prow * kPartStride;
}

namespace nkv {

int fill_attend_params(const char* who, const nkv_store* st, int layer0, int num_layers,
                       const uint16_t* q, int64_t q_layer_stride, int tq, const uint16_t* k_new,
                       const uint16_t* v_new, int64_t kv_layer_stride, int n_chunk, int write_slot,
                       const int32_t* ids, int64_t ids_layer_stride, int n_hist,
                       const uint8_t* allowed, int64_t allowed_layer_stride, int sink_len,
                       int ring_base, int rec_lo, int rec_len,
                       float scale, int splits, float* partial_ws, uint16_t* out,
                       AttendParams* pp) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  const int G = st->num_heads / st->num_kv_heads;
  const int R = st->recent_tokens;
  NKV_CHECK_ARG(q != nullptr && out != nullptr, "%s: q and out must be non-NULL", who);
  NKV_CHECK_ARG(tq >= 1 && tq <= 65536, "%s: tq must be in [1, 65536] (got %d)", who, tq);
  NKV_CHECK_ARG(n_hist >= 0 && n_hist <= 4096, "%s: n_hist must be in [0, 4096] (got %d)", who, n_hist);
  NKV_CHECK_ARG(n_hist == 0 || ids != nullptr, "%s: ids is NULL but n_hist=%d", who, n_hist);
  NKV_CHECK_ARG(sink_len >= 0 && sink_len <= st->sink_tokens, "%s: sink_len %d outside [0, %d]",
                who, sink_len, st->sink_tokens);
  NKV_CHECK_ARG(rec_len >= 0 && rec_lo >= 0 && rec_lo + rec_len <= R,
                "%s: recent range [%d, %d) outside [0, %d)", who, rec_lo, rec_lo + rec_len, R);
  NKV_CHECK_ARG(ring_base >= 0 && ring_base < R, "%s: ring_base %d outside [0, %d)", who, ring_base, R);
  NKV_CHECK_ARG(n_chunk == 0 || n_chunk == tq,
                "%s: the causal chunk must have one token per query (n_chunk=%d, tq=%d)", who, n_chunk, tq);
  NKV_CHECK_ARG(n_chunk == 0 || (k_new != nullptr && v_new != nullptr),
                "%s: k_new/v_new are NULL but n_chunk=%d", who, n_chunk);
  NKV_CHECK_ARG(write_slot < R, "%s: write_slot %d outside the ring", who, write_slot);
  NKV_CHECK_ARG(write_slot < 0 || n_chunk >= 1, "%s: write_slot needs a new token (n_chunk >= 1)", who);
  if (write_slot >= 0 && rec_len > 0) {
    // the slot being written must not be one the call reads
    const int lp = ((write_slot - ring_base) % R + R) % R;
    NKV_CHECK_ARG(lp < rec_lo || lp >= rec_lo + rec_len,
                  "%s: write_slot %d lies inside the attended recent window", who, write_slot);
  }
  NKV_CHECK_ARG(splits >= 0 && splits <= 64,
                "%s: splits must be in [0, 64] (got %d; 0 = stream form / tiered plan)", who, splits);
  NKV_CHECK_ARG(splits == 1 || partial_ws != nullptr, "%s: splits != 1 needs partial_ws", who);
  const int n_sink_seg = (sink_len + kBlock - 1) / kBlock;
  const int n_rec_seg = rec_len > 0 ? (R + kBlock - 1) / kBlock : 0;
  const int n_chunk_seg = (n_chunk + kBlock - 1) / kBlock;
  const int nseg = n_hist + n_sink_seg + n_rec_seg + n_chunk_seg;
  NKV_CHECK_ARG(nseg >= 1, "%s: nothing to attend", who);

  AttendParams& p = *pp;
  const int64_t hist_ls = static_cast<int64_t>(st->num_kv_heads) * st->cap_blocks * kBlock * kHeadDim;
  const int64_t elem = st->kv_format == NKV_KV_BF16 ? 2 : 1;
  p.hist_k = static_cast<const char*>(st->hist_k) + layer0 * hist_ls * elem;
  p.hist_v = static_cast<const char*>(st->hist_v) + layer0 * hist_ls * elem;
  p.hist_ls = hist_ls;
  p.sink_ls = static_cast<int64_t>(st->num_kv_heads) * st->sink_tokens * kHeadDim;
  p.sink_k = st->sink_k ? static_cast<const uint16_t*>(st->sink_k) + layer0 * p.sink_ls : nullptr;
  p.sink_v = st->sink_v ? static_cast<const uint16_t*>(st->sink_v) + layer0 * p.sink_ls : nullptr;
  p.rec_ls = static_cast<int64_t>(st->num_kv_heads) * R * kHeadDim;
  p.rec_k = static_cast<uint16_t*>(st->recent_k) + layer0 * p.rec_ls;
  p.rec_v = static_cast<uint16_t*>(st->recent_v) + layer0 * p.rec_ls;
  p.k_scale = st->k_scale ? st->k_scale + static_cast<int64_t>(layer0) * st->num_kv_heads * kHeadDim : nullptr;
  p.v_scale = st->v_scale ? st->v_scale + static_cast<int64_t>(layer0) * st->num_kv_heads * st->cap_blocks : nullptr;
  const int64_t ts_ls = static_cast<int64_t>(st->num_kv_heads) * st->cap_blocks * kBlock;
  p.k_tscale = st->k_tscale ? st->k_tscale + layer0 * ts_ls : nullptr;
  p.v_tscale = st->v_tscale ? st->v_tscale + layer0 * ts_ls : nullptr;
  p.q = q;
  p.q_ls = q_layer_stride;
  p.k_new = k_new;
  p.v_new = v_new;
  p.kv_ls = kv_layer_stride;
  p.ids = ids;
  p.ids_ls = ids_layer_stride;
  NKV_CHECK_ARG(allowed_layer_stride == 0 || allowed_layer_stride >= static_cast<int64_t>(tq) * n_hist,
                "%s: allowed_layer_stride %lld is neither 0 (shared) nor >= tq * n_hist", who,
                static_cast<long long>(allowed_layer_stride));
  p.allowed = allowed;
  p.allowed_ls = allowed ? allowed_layer_stride : 0;
  p.partial = partial_ws;
  p.out = out;
  p.hkv = st->num_kv_heads;
  p.G = G;
  p.cap = st->cap_blocks;
  p.S = st->sink_tokens;
  p.R = R;
  p.tq = tq;
  p.qpg = 1;
  p.nqg = tq;
  p.n_chunk = n_chunk;
  p.write_slot = write_slot;
  p.n_hist = n_hist;
  p.sink_len = sink_len;
  p.ring_base = ring_base;
  p.ring_start = nullptr;
  p.rec_lo = rec_lo;
  p.rec_len = rec_len;
  p.n_sink_seg = n_sink_seg;
  p.n_rec_seg = n_rec_seg;
  p.nseg = nseg;
  p.splits = splits;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.causal_off = 0;
  p.tok_mask = nullptr;
  p.zero_keys = nullptr;
  p.zero_n = 0;
  p.ids_tile_ls = 0;
  p.sel_tile = 0;
  p.stream_wpg = 0;
  p.nlayers = num_layers;
  p.wide_ga = p.wide_sa = p.wide_sb = 0;
  return NKV_OK;
}

}  // namespace nkv

namespace nkv {
int attend_impl(const nkv_store* st, int layer0, int num_layers, const uint16_t* q, int64_t q_layer_stride, int tq,
                const uint16_t* k_new, const uint16_t* v_new, int64_t kv_layer_stride, int n_chunk, int write_slot,
                const int32_t* ids, int64_t ids_layer_stride, int n_hist, const uint8_t* allowed,
                int64_t allowed_layer_stride, int sink_len, int ring_base, int rec_lo, int rec_len, float scale,
                int splits, float* partial_ws, uint16_t* out, uint32_t* zero_keys, int zero_n, void* stream) {
  AttendParams p;
  const int rc = fill_attend_params("nkv_attend", st, layer0, num_layers, q, q_layer_stride, tq, k_new,
                                    v_new, kv_layer_stride, n_chunk, write_slot, ids, ids_layer_stride,
                                    n_hist, allowed, allowed_layer_stride, sink_len, ring_base, rec_lo,
                                    rec_len, scale, splits, partial_ws, out, &p);
  if (rc != NKV_OK) return rc;
  p.zero_keys = zero_keys;
  p.zero_n = zero_n;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int lrc = launch_grouped(st->num_kv_heads, st->kv_format, num_layers, tq, p, s);
  return lrc != NKV_OK ? lrc : launch_status("nkv_attend");
}
}  // namespace nkv

extern "C" int nkv_attend(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                          int64_t q_layer_stride, int tq, const uint16_t* k_new,
                          const uint16_t* v_new, int64_t kv_layer_stride, int n_chunk,
                          int write_slot, const int32_t* ids, int64_t ids_layer_stride,
                          int n_hist, const uint8_t* allowed, int64_t allowed_layer_stride,
                          int sink_len, int ring_base, int rec_lo, int rec_len, float scale, int splits,
                          float* partial_ws, uint16_t* out, void* stream) {
  return attend_impl(st, layer0, num_layers, q, q_layer_stride, tq, k_new, v_new, kv_layer_stride, n_chunk,
                     write_slot, ids, ids_layer_stride, n_hist, allowed, allowed_layer_stride, sink_len, ring_base,
                     rec_lo, rec_len, scale, splits, partial_ws, out, nullptr, 0, stream);
}

extern "C" int nkv_decode_step_ring(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                                    const uint16_t* k_new, const uint16_t* v_new, int nblocks,
                                    const int32_t* protected_ids, int n_protected, int k, int n_hist,
                                    int sink_len, int32_t* ring_start, float scale, int splits,
                                    uint32_t* score_keys, int32_t* out_ids, float* partial_ws, uint16_t* out,
                                    void* stream) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_ARG(q != nullptr && k_new != nullptr && v_new != nullptr && score_keys != nullptr &&
                    out_ids != nullptr && out != nullptr && ring_start != nullptr,
                "nkv_decode_step_ring: q, k_new, v_new, score_keys, out_ids, out and ring_start must be non-NULL");
  NKV_CHECK_ARG(n_hist >= 1 && n_hist <= k, "nkv_decode_step_ring: n_hist must be in [1, k] (got %d, k=%d)", n_hist,
                k);
  const int R = st->recent_tokens;
  NKV_CHECK_ARG(R >= 2, "nkv_decode_step_ring: needs a recent window of at least 2 tokens");
  const int64_t q_ls = static_cast<int64_t>(st->num_heads) * kHeadDim;
  const int64_t kv_ls = static_cast<int64_t>(st->num_kv_heads) * kHeadDim;
  // The full window: the R - 1 recent tokens before the write slot, then the
  // new token.  Write slot 0 / base 1 stand in for the host checks; the
  // kernel reads each layer's ring start from device memory.  Checked before
  // the selection is enqueued (its step form leaves the keys for the
  // attention launch to clear).
  AttendParams p;
  rc = fill_attend_params("nkv_decode_step_ring", st, layer0, num_layers, q, q_ls, 1, k_new, v_new, kv_ls, 1, 0,
                          out_ids, k, n_hist, nullptr, 0, sink_len, 1, 0, R - 1, scale, splits, partial_ws, out, &p);
  if (rc != NKV_OK) return rc;
  rc = select_impl(st, layer0, num_layers, q, q_ls, 1, 0, nblocks, protected_ids, n_protected, k,
                   NKV_ORDER_SCORE_DESC, score_keys, nullptr, out_ids, nullptr, true, stream);
  if (rc != NKV_OK) return rc;
  const bool step_keys = select_step_form(1, n_protected, nblocks);
  p.ring_start = ring_start;
  if (step_keys) {
    p.zero_keys = score_keys;
    p.zero_n = nblocks;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  rc = launch_grouped(st->num_kv_heads, st->kv_format, num_layers, 1, p, s);   // with splits != 1 the merge advances the ring
  if (rc != NKV_OK) return rc;
  if (splits == 1)
    hipLaunchKernelGGL(ring_advance_kernel, dim3((num_layers + kWave - 1) / kWave), dim3(kWave), 0, s, ring_start,
                       num_layers, R);
  return launch_status("nkv_decode_step_ring");
}

// Caller-packed keys: every key is a chunk key (token-major [s_len][Hkv][D]),
// visible to query t iff key - causal_from <= t and mask[t][key] == 0.
// Queries whose rows exceed one 16-row MFMA tile per KV head go to the
// matrix-core kernel, the others to the few-query kernel.
namespace {
bool packed_uses_prefill(int tq, int G) { return tq * G > kMaxRows; }
}  // namespace

extern "C" int64_t nkv_attend_packed_workspace_floats(int num_heads, int num_kv_heads, int tq, int splits) {
  if (num_kv_heads < 1 || num_heads < num_kv_heads || num_heads % num_kv_heads != 0 || tq < 1 || splits < 1)
    return 0;
  if (packed_uses_prefill(tq, num_heads / num_kv_heads))
    return nkv_prefill_workspace_floats(1, num_kv_heads, num_heads, tq, splits);
  return splits == 1 ? 0 : nkv_attend_workspace_floats(1, num_kv_heads, num_heads, tq, splits);
}

extern "C" int nkv_attend_packed(int num_heads, int num_kv_heads, const uint16_t* q, int tq, const uint16_t* k,
                                 const uint16_t* v, int s_len, int causal_from, const uint8_t* mask, float scale,
                                 int splits, float* partial_ws, uint16_t* out, void* stream) {
  NKV_CHECK_ARG(num_kv_heads >= 1 && num_heads >= num_kv_heads && num_heads % num_kv_heads == 0,
                "nkv_attend_packed: num_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_heads,
                num_kv_heads);
  const int G = num_heads / num_kv_heads;
  NKV_CHECK_SUPPORTED(G == 1 || G == 2 || G == 4 || G == 8 || G == 16,
                      "nkv_attend_packed: query heads per KV head must be 1, 2, 4, 8 or 16 (got %d)", G);
  NKV_CHECK_ARG(q != nullptr && k != nullptr && v != nullptr && out != nullptr,
                "nkv_attend_packed: q, k, v and out must be non-NULL");
  NKV_CHECK_ARG(tq >= 1 && tq <= 65536, "nkv_attend_packed: tq must be in [1, 65536] (got %d)", tq);
  NKV_CHECK_ARG(s_len >= 1 && s_len <= (1 << 20), "nkv_attend_packed: s_len must be in [1, 2^20] (got %d)", s_len);
  NKV_CHECK_ARG(causal_from >= 0, "nkv_attend_packed: causal_from must be >= 0 (got %d)", causal_from);
  NKV_CHECK_ARG(splits >= 1 && splits <= 64, "nkv_attend_packed: splits must be in [1, 64] (got %d)", splits);
  NKV_CHECK_ARG(splits == 1 || partial_ws != nullptr, "nkv_attend_packed: splits > 1 needs partial_ws");
  AttendParams p = {};
  p.q = q;
  p.k_new = k;
  p.v_new = v;
  p.partial = partial_ws;
  p.out = out;
  p.hkv = num_kv_heads;
  p.G = G;
  p.cap = 1;
  p.S = 0;
  p.R = 1;
  p.tq = tq;
  p.qpg = 1;
  p.nqg = tq;
  p.n_chunk = s_len;
  p.write_slot = -1;
  p.ring_start = nullptr;
  p.nseg = (s_len + kBlock - 1) / kBlock;
  p.splits = splits;
  p.scale_log2 = scale * 1.4426950408889634f;
  // keys past causal_from + tq - 1 are hidden from every query
  p.causal_off = causal_from < s_len ? causal_from : s_len;
  p.tok_mask = mask;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int rc = packed_uses_prefill(tq, G) ? launch_prefill(num_kv_heads, NKV_KV_BF16, 1, tq, p, s)
                                            : launch_grouped(num_kv_heads, NKV_KV_BF16, 1, tq, p, s);
  return rc != NKV_OK ? rc : launch_status("nkv_attend_packed");
}
