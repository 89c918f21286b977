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
// Per 64-key segment:
//   * the segment is staged through registers into an LDS buffer (double
//     buffered, one barrier per segment; the next segment's global loads are
//     in flight while the current one is computed): K as 64 rows x 256 B with
//     the 16-byte chunk index XOR-swizzled by the row, V transposed to 128
//     rows (dims) x 64 keys, keys permuted inside a row so that one 16-byte
//     LDS read returns the 8 keys an MFMA lane needs;
//   * S^T = K . Q^T: v_mfma_f32_16x16x32_bf16, A = 16 keys x 32 dims from LDS,
//     B = 32 dims x 16 columns held in registers for the whole kernel;
//   * online softmax in fp32 per column (exp2, scale folded in); each lane's
//     column is fixed, so the running max and the rescale stay in the lane;
//   * O^T += V^T . P^T: A = 16 dims x 32 keys from the transposed V tile,
//     B = the lane's own probabilities rounded to bf16 (the 32-key
//     contraction index is ordered as the S^T accumulator holds the keys, so
//     P never leaves the registers).
//
// The reference runs this as flash-attention over the packed
// [selected | sink | recent | chunk] keys with bottom-right causal masking
// (nanovllm/sparse/m12_runtime.py:592-651, :809-839); the fp32 masked path
// (:875-896) is the same function.
#include "nkv_attend_common.h"

namespace nkv {
namespace {
using namespace attend_detail;

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;     // 256
constexpr int kPfCols = 128;                     // (token, head) columns per workgroup
constexpr int kKTileBytes = kBlock * kHeadDim * 2;
constexpr int kBufBytes = 2 * kKTileBytes;       // K tile + transposed V tile

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Byte offset of 16-byte chunk `chunk` (dims 8 chunk .. +8) of key row `row`.
__device__ __forceinline__ int k_off(int row, int chunk) {
  return row * 256 + ((chunk ^ (row & 15)) << 4);
}

// Byte offset of chunk `chunk` (8 permuted keys) of transposed-V row `dim`.
// Key k sits in chunk 4 (k / 32) + (k % 16) / 4 at element 4 ((k % 32) / 16) + k % 4.
__device__ __forceinline__ int vt_off(int dim, int chunk) {
  const int swz = (dim & 7) ^ ((dim >> 2) & 6);
  return kKTileBytes + dim * 128 + ((chunk ^ swz) << 4);
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
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

// One segment in flight between its global loads and its LDS store.
struct Stage {
  u32x4 k[4];   // K rows kr0 + 16 j, dims 8 kc .. +8 (int8: 8 bytes in .x/.y)
  u32x4 v[4];   // V keys vkey0 + j, dims 8 vdg .. +8
  float ks[4];  // int8 per-token scales of those K rows
  float vs[4];  // int8 per-token scales of those V keys (per-block: vs[0])
};

// Thread roles in the staging (tid = 0..255):
//   K: rows (tid >> 4) + 16 j, j < 4, 16-byte chunk tid & 15;
//   V: keys vkey0 + j, j < 4, dims 8 vdg .. +8, written transposed as 8 rows
//      of 4 keys; the mapping makes each quarter-wave's 8-byte LDS writes
//      cover all 32 banks.
struct VRole {
  int key0, dg, chunk, half;
};

__device__ __forceinline__ VRole v_role(int tid) {
  const int wave = tid >> 6;
  const int u = tid & 15;
  const int quarter = (tid >> 4) & 3;
  const int lg = 2 * (wave & 1) + (u & 1);
  const int half = (u >> 1) & 1;
  VRole r;
  r.dg = (u >> 2) + 4 * quarter;
  r.chunk = 4 * (wave >> 1) + lg;
  r.half = half;
  r.key0 = 32 * (wave >> 1) + 16 * half + 4 * lg;
  return r;
}

template <int FMT>
__device__ __forceinline__ void load_stage(const AttendParams& p, const Seg& g, int lh, int tid,
                                           const VRole& vr, Stage& st) {
  const int last = g.len - 1;
  const int kr0 = tid >> 4;
  const int kc = tid & 15;
  if (FMT != NKV_KV_BF16 && g.type == kSegHist) {
    const int64_t tb = (static_cast<int64_t>(lh) * p.cap + g.blk) * kBlock;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = min(kr0 + 16 * j, last);
      const int key = min(vr.key0 + j, last);
      const u32x2 x = *reinterpret_cast<const u32x2*>(g.kbase + row * g.rowb + kc * 8);
      const u32x2 y = *reinterpret_cast<const u32x2*>(g.vbase + key * g.rowb + vr.dg * 8);
      st.k[j] = u32x4{x[0], x[1], 0u, 0u};
      st.v[j] = u32x4{y[0], y[1], 0u, 0u};
      if (FMT == NKV_KV_INT8_TOKEN) {
        st.ks[j] = f16_bits_to_f32(p.k_tscale[tb + row]);
        st.vs[j] = f16_bits_to_f32(p.v_tscale[tb + key]);
      }
    }
    if (FMT == NKV_KV_INT8_CHANNEL) st.vs[0] = p.v_scale[static_cast<int64_t>(lh) * p.cap + g.blk];
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      st.k[j] = *reinterpret_cast<const u32x4*>(g.kbase + min(kr0 + 16 * j, last) * g.rowb + kc * 16);
      st.v[j] = *reinterpret_cast<const u32x4*>(g.vbase + min(vr.key0 + j, last) * g.rowb + vr.dg * 16);
    }
  }
}

template <int FMT>
__device__ __forceinline__ void store_stage(char* buf, Stage& st, bool int8_seg, const float (&kch)[8],
                                            int tid, const VRole& vr) {
  const int kr0 = tid >> 4;
  const int kc = tid & 15;
  if (FMT != NKV_KV_BF16 && int8_seg) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float ksc[8], vsc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ksc[e] = FMT == NKV_KV_INT8_CHANNEL ? kch[e] : st.ks[j];
        vsc[e] = FMT == NKV_KV_INT8_CHANNEL ? st.vs[0] : st.vs[j];
      }
      st.k[j] = dequant8(st.k[j][0], st.k[j][1], ksc);
      st.v[j] = dequant8(st.v[j][0], st.v[j][1], vsc);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(buf + k_off(kr0 + 16 * j, kc)) = st.k[j];
  // transpose: dim 8 dg + e gets the 4 keys' e-th values
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
    const int wi = e >> 1;
    const uint32_t lo = __builtin_amdgcn_perm(st.v[1][wi], st.v[0][wi], sel);
    const uint32_t hi = __builtin_amdgcn_perm(st.v[3][wi], st.v[2][wi], sel);
    *reinterpret_cast<u32x2*>(buf + vt_off(8 * vr.dg + e, vr.chunk) + vr.half * 8) = u32x2{lo, hi};
  }
}

// Whether any (key, column) of segment g may be invisible to the workgroup's
// tokens t0.. (otherwise the mask pass is skipped).
__device__ __forceinline__ bool needs_mask(const AttendParams& p, const Seg& g, int t0) {
  switch (g.type) {
    case kSegHist: return g.vlen < kBlock || p.allowed != nullptr;
    case kSegSink: return g.len < kBlock;
    case kSegRecent: return !(p.rec_len == p.R && g.len == kBlock);
    default: return g.len < kBlock || g.off + kBlock - 1 > t0;
  }
}

template <int FMT>
__global__ __launch_bounds__(kPfThreads, 2) void prefill_kernel(const AttendParams p, int nqt) {
  __shared__ __attribute__((aligned(16))) char lds[2 * kBufBytes];

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
  const VRole vr = v_role(tid);

  float kch[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) kch[e] = 1.0f;
  if (FMT == NKV_KV_INT8_CHANNEL) {
    const float* ks = p.k_scale + static_cast<int64_t>(lh) * kHeadDim + (tid & 15) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) kch[e] = ks[e];
  }

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

  const int n_chunk_seg = p.n_chunk > 0 ? t_last / kBlock + 1 : 0;
  const int nseg = p.n_hist + p.n_sink_seg + p.n_rec_seg + n_chunk_seg;

  Stage stg;
  Seg nxt = make_seg<FMT>(p, layer, h, 0);
  load_stage<FMT>(p, nxt, lh, tid, vr, stg);
  store_stage<FMT>(lds, stg, FMT != NKV_KV_BF16 && nxt.type == kSegHist, kch, tid, vr);
  __syncthreads();

  for (int s = 0; s < nseg; ++s) {
    const Seg cur = nxt;
    const bool more = s + 1 < nseg;
    if (more) {
      nxt = make_seg<FMT>(p, layer, h, s + 1);
      load_stage<FMT>(p, nxt, lh, tid, vr, stg);
    }
    const char* buf = lds + (s & 1) * kBufBytes;

    // ---- S^T = K . Q^T -----------------------------------------------------
    // S[kt][ct][e]: key 16 kt + 4 lg + e, column (ct, ln)
    f32x4 S[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) S[kt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(buf + k_off(16 * kt + ln, 4 * ks + lg));
        S[kt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[0][ks], S[kt][0], 0, 0, 0);
        S[kt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[1][ks], S[kt][1], 0, 0, 0);
      }
    }

    // ---- visibility ---------------------------------------------------------
    if (needs_mask(p, cur, t0)) {
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const int t = tcol[ct];
        bool col_ok = true;
        if (cur.type == kSegHist && p.allowed != nullptr)
          col_ok = p.allowed[static_cast<int64_t>(min(t, p.tq - 1)) * p.n_hist + cur.u] != 0;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = 16 * kt + 4 * lg + e;
            bool ok = col_ok && key < cur.vlen;
            if (cur.type == kSegRecent) {
              int lp = cur.off + key - p.ring_base;
              if (lp < 0) lp += p.R;
              ok = ok && static_cast<unsigned>(lp - p.rec_lo) < static_cast<unsigned>(p.rec_len);
            } else if (cur.type == kSegChunk) {
              ok = ok && cur.off + key <= t;
            }
            if (!ok) S[kt][ct][e] = -INFINITY;
          }
        }
      }
    }

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
      const float m_new = fmaxf(m_run[ct], mx * p.scale_log2);
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
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(buf + vt_off(16 * dt + ln, 4 * k2 + lg));
        acc[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[0], acc[dt][0], 0, 0, 0);
        acc[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[1], acc[dt][1], 0, 0, 0);
      }
    }

    if (more) store_stage<FMT>(lds + ((s + 1) & 1) * kBufBytes, stg, FMT != NKV_KV_BF16 && nxt.type == kSegHist,
                               kch, tid, vr);
    __syncthreads();
  }

  // ---- normalise and store: acc[dt][ct][i] = dim 16 dt + 4 lg + i -----------
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    float l = l_run[ct];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const int t = tcol[ct];
    if (t <= t_last) {
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

}  // namespace
}  // namespace nkv

using namespace nkv;

extern "C" int nkv_prefill_attend(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                                  int64_t q_layer_stride, int tq, const uint16_t* k_new,
                                  const uint16_t* v_new, int64_t kv_layer_stride, const int32_t* ids,
                                  int64_t ids_layer_stride, int n_hist, const uint8_t* allowed,
                                  int sink_len, int ring_base, int rec_lo, int rec_len, float scale,
                                  uint16_t* out, void* stream) {
  AttendParams p;
  const int rc = fill_attend_params("nkv_prefill_attend", st, layer0, num_layers, q, q_layer_stride, tq,
                                    k_new, v_new, kv_layer_stride, tq, -1, ids, ids_layer_stride, n_hist,
                                    allowed, sink_len, ring_base, rec_lo, rec_len, scale, 1, nullptr, out, &p);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_SUPPORTED(p.G >= 1 && kPfCols % p.G == 0,
                      "nkv_prefill_attend: query heads per KV head (%d) must divide %d", p.G, kPfCols);
  const int tpw = kPfCols / p.G;
  const int nqt = (tq + tpw - 1) / tpw;
  const dim3 grid(nqt * st->num_kv_heads, num_layers);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (st->kv_format) {
    case NKV_KV_BF16: hipLaunchKernelGGL(prefill_kernel<NKV_KV_BF16>, grid, dim3(kPfThreads), 0, s, p, nqt); break;
    case NKV_KV_INT8_CHANNEL:
      hipLaunchKernelGGL(prefill_kernel<NKV_KV_INT8_CHANNEL>, grid, dim3(kPfThreads), 0, s, p, nqt);
      break;
    case NKV_KV_INT8_TOKEN:
      hipLaunchKernelGGL(prefill_kernel<NKV_KV_INT8_TOKEN>, grid, dim3(kPfThreads), 0, s, p, nqt);
      break;
    default: NKV_CHECK_SUPPORTED(false, "nkv_prefill_attend: unknown kv_format %d", st->kv_format);
  }
  return launch_status("nkv_prefill_attend");
}
