// Streaming few-query attention (the decode layer-step's gather + attention)
// on gfx950: a persistent, stream-K kernel that keeps HBM busy.
//
// The work is the flat list of (pair, segment) tiles, pair = (layer, KV
// head), segments as in nkv_attend.hip (selected history blocks read in
// place, sink, physical ring pieces masked to the logical window, the causal
// chunk).  Workgroup i of W takes the contiguous range
// [i T / W, (i + 1) T / W) of the T = pairs x segments tiles, so every
// workgroup streams the same number of bytes whatever the layer / head
// boundaries.
//
// Each workgroup (4 wavefronts, one per SIMD, all of a CU's LDS) runs a ring
// of LDS stages filled by direct global -> LDS copies (buffer_load ... lds):
// all but one of the stages are in flight while one is
// computed, with no registers held for them.  A stage holds the segment's K
// and V tiles (stage.h layout) and the query rows of its pair, so every copy
// issues the same number of vector-memory operations per wavefront and the
// wait for a stage is a fixed count.
//
// Per segment all four wavefronts compute S^T = K . Q^T (MFMA, 64 keys x up
// to 16 NCT query rows) and the online softmax (identical in every wave); the
// P.V product is split by output dims: wavefront w owns dims 32w .. 32w+31
// (V^T from the transposing LDS read, P^T from the lane's own probabilities
// as bf16 hi + lo parts, so P.V keeps fp32 accuracy).  So no cross-wave merge is needed: at the end of its part
// of a pair each wavefront writes its dims of a partial (m, l, acc) record,
// slot pair + i, and attend_stream_merge combines the records of a pair.
#include <type_traits>

#include "nkv_stage.h"

namespace nkv {
namespace {
using namespace attend_detail;
using namespace stage;

constexpr int kDcThreads = 256;

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt
// in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
constexpr int vm_wait_imm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }
// waits for this wave's LDS operations only
constexpr int kLgkmZero = 15 | (3 << 14) | (7 << 4);

// Query-row area appended to each stage: 16 rows x 256 B per column tile,
// 16-byte chunk c of row r at position c ^ (r & 15) (as the K tile).
template <int NCT>
constexpr int stage_bytes() {
  return kBufBytes + NCT * 16 * 256;
}

struct StreamWork {
  int total;       // pairs x segments (< 2^31, checked by the launcher)
  int npair;
  int nseg;
  int nwg;
  int rows;        // query rows of a pair (tq x G)
};

// Copies the q rows of pair (layer, h) into the stage's query area.  Row
// c = 16 ct + r is (token c / G, head h G + c % G); rows >= rows read as zero
// (offset past the descriptor's range).  Wavefront w copies rows 4 w' .. 4 w' + 3
// for w' = w, w + 4 (NCT = 2).
template <int NCT>
__device__ __forceinline__ void dma_query(const AttendParams& p, const StreamWork& w, int layer, int h,
                                          char* qarea, int wave, int lane, bool live) {
  const int hq = p.hkv * p.G;
  const int64_t qbytes = live ? static_cast<int64_t>(p.tq) * hq * kHeadDim * 2 : 0;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.q + p.q_ls * layer), 0, static_cast<int>(qbytes), kRsrcWord3);
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int rblk = wave + 4 * i;              // 4-row block of the area
    const int row = 4 * rblk + (lane >> 4);      // 0 .. 16 NCT - 1
    const int c = (lane & 15) ^ (row & 15);      // global chunk landing at position lane & 15
    const int t = row / p.G;
    const int hh = h * p.G + row % p.G;
    const int off = row < w.rows ? (t * hq + hh) * kHeadDim * 2 + c * 16 : 0x7ffffff0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(qarea + rblk * 1024), 16, off, 0, 0, 0);
  }
}

// Ring depth: 4 stages for up to 16 query rows (4 x 36 KiB), 3 for up to 32
// (3 x 40 KiB), plus the workgroup's block ids.
template <int NCT>
constexpr int ring_stages() {
  return NCT == 1 ? 4 : 3;
}
constexpr int kIdsMax = 512;   // tiles per workgroup range (block ids staged in LDS)

template <int NCT>
__global__ __launch_bounds__(kDcThreads, 1) void attend_stream_kernel(const AttendParams p, const StreamWork w) {
  constexpr int kSB = stage_bytes<NCT>();
  constexpr int kNS = ring_stages<NCT>();
  constexpr int kOps = 8 + NCT;   // vector-memory operations per wavefront per stage copy
  // one object per stage, so that the compiler can tell the stage being read
  // from the stages the asynchronous copies write
  __shared__ __attribute__((aligned(16))) char st0[kSB];
  __shared__ __attribute__((aligned(16))) char st1[kSB];
  __shared__ __attribute__((aligned(16))) char st2[kSB];
  __shared__ __attribute__((aligned(16))) char st3[kNS > 3 ? kSB : 16];
  __shared__ int ids_lds[kIdsMax];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int ln = lane & 15;
  const int lg = lane >> 4;
  const int g0 = static_cast<int>(static_cast<int64_t>(blockIdx.x) * w.total / w.nwg);
  const int g1 = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * w.total / w.nwg);
  if (g0 >= g1) return;

  // tile index -> (layer, KV head, segment); uniform, in scalar registers
  auto seg_of = [&](int g, int* layer, int* h, int* s) __attribute__((always_inline)) {
    const int pair = __builtin_amdgcn_readfirstlane(g / w.nseg);
    *s = __builtin_amdgcn_readfirstlane(g - pair * w.nseg);
    *layer = __builtin_amdgcn_readfirstlane(pair / p.hkv);
    *h = __builtin_amdgcn_readfirstlane(pair - *layer * p.hkv);
  };

  // block ids of the range's history tiles -> LDS (the copies below are
  // asynchronous memory operations the compiler cannot see past, which would
  // otherwise turn every id lookup into a vector load and a full wait)
  for (int i = tid; i < g1 - g0; i += kDcThreads) {
    const int g = g0 + i;
    const int pair = g / w.nseg;
    const int sg = g - pair * w.nseg;
    const int layer = pair / p.hkv;
    ids_lds[i] = sg < p.n_hist ? p.ids[static_cast<int64_t>(layer) * p.ids_ls + sg] : 0;
  }
  __syncthreads();

  // ---- loop-invariant LDS offsets (bytes, within a stage) --------------------
  int koff[4];   // K (and q) read: row 16 kt + ln, chunk 4 ks + lg (kt -> + 4096 kt)
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = ln * 256 + ((((4 * ks + lg) ^ ln) & 15) << 4);
  // V transposing read for this wave's dims 16 dt + ..., dt = 2 wave + d
  int vtr[2];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const int q = (2 * wave + d) & 3;
    vtr[d] = kTileBytes + (4 * lg + (ln >> 2)) * 256 + ((2 * (q ^ (ln >> 2)) + ((ln & 3) >> 1)) << 4) +
             8 * (ln & 1) + ((2 * wave + d) >> 2) * 128;
  }
  int kx[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kx[i] = (ln ^ ((4 * i + lg) & 15)) << 4;
  const int vx = (ln ^ (2 * lg)) << 4;

  auto stage_ptr = [&](auto kk) __attribute__((always_inline)) -> char* {
    constexpr int K = decltype(kk)::value;
    return K == 0 ? st0 : K == 1 ? st1 : K == 2 ? st2 : st3;
  };
  auto seg_at = [&](int g, int layer, int h, int s) __attribute__((always_inline)) {
    return make_seg_blk<NKV_KV_BF16>(p, layer, h, s, __builtin_amdgcn_readfirstlane(ids_lds[g - g0]));
  };
  // Every tile slot issues its copies, also past the range (an empty
  // descriptor: same instruction count, nothing read), so that the number of
  // copies younger than any stage is a constant and so is every wait.
  auto issue = [&](int g, char* st) __attribute__((always_inline)) {
    const bool live = g < g1;
    const int gc = live ? g : g1 - 1;
    int layer, h, s;
    seg_of(gc, &layer, &h, &s);
    const Seg sg = seg_at(gc, layer, h, s);
    dma_segment(sg, st, wave, lane, kx, vx, live);
    dma_query<NCT>(p, w, layer, h, st + kBufBytes, wave, lane, live);
  };

  // prologue: kNS - 1 tiles in flight
  issue(g0, st0);
  issue(g0 + 1, st1);
  if (kNS > 3) issue(g0 + 2, st2);

  float m_run[NCT], l_run[NCT];
  f32x4 acc[2][NCT];
  auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      m_run[ct] = -INFINITY;
      l_run[ct] = 0.0f;
      acc[0][ct] = acc[1][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  reset();

  // one tile on stage K (K = tile index mod kNS, a compile-time constant)
  auto body = [&](auto kk, int g) __attribute__((always_inline)) {
    constexpr int K = decltype(kk)::value;
    // tile g has landed once at most the kNS - 2 younger copies are
    // outstanding; then a bare barrier (a memory fence would wait for every copy)
    __builtin_amdgcn_s_waitcnt(vm_wait_imm((kNS - 2) * kOps));
    __builtin_amdgcn_s_waitcnt(kLgkmZero);
    __builtin_amdgcn_s_barrier();
    // the stage of tile g - 1 is free again (every wave is past its compute)
    issue(g + kNS - 1, stage_ptr(std::integral_constant<int, (K + kNS - 1) % kNS>{}));

    if (g >= g1) return;   // a slot past the range: only its (empty) copy was issued
    int layer, h, s;
    seg_of(g, &layer, &h, &s);
    const Seg cur = seg_at(g, layer, h, s);
    const char* st = stage_ptr(kk);
    const char* qa = st + kBufBytes;
    // ---- S^T = K . Q^T: S[kt][ct][e] = key 16 kt + 4 lg + e, column 16 ct + ln
    f32x4 S[4][NCT];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) S[kt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 bq[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) bq[ct] = *reinterpret_cast<const bf16x8*>(qa + ct * 4096 + koff[ks]);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(st + kt * 4096 + koff[ks]);
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          S[kt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[ct], S[kt][ct], 0, 0, 0);
      }
    }

    // ---- visibility (history ids out of range, partial sink / ring / chunk)
    const bool full = cur.type == kSegHist ? cur.vlen == kBlock
                    : cur.type == kSegSink ? cur.len == kBlock
                    : cur.type == kSegRecent ? (p.rec_len == p.R && cur.len == kBlock)
                    : false;
    if (!full) {
      if (cur.type == kSegRecent) {
        int a = (cur.off - p.ring_base - p.rec_lo) % p.R;
        a = a < 0 ? a + p.R : a;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = 16 * kt + 4 * lg + e;
            int x = a + key;
            x -= p.R & ((p.R - 1 - x) >> 31);
            const float bound = vis_bound(max(key - (cur.vlen - 1), x - (p.rec_len - 1)));
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) S[kt][ct][e] = fminf(S[kt][ct][e], bound);
          }
      } else {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          int thr = cur.vlen - 1;
          if (cur.type == kSegChunk) thr = min(thr, (16 * ct + ln) / p.G - cur.off);
          const int base = 4 * lg - thr;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int e = 0; e < 4; ++e) S[kt][ct][e] = fminf(S[kt][ct][e], vis_bound(base + 16 * kt + e));
        }
      }
    }

    // ---- online softmax (fp32, lazy reference max) ---------------------------
    float alpha[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      float mx = S[0][ct][0];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, S[kt][ct][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
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
#pragma unroll
      for (int d = 0; d < 2; ++d) acc[d][ct] *= alpha[ct];
    }

    // ---- O^T += V^T . P^T for this wave's 32 dims ----------------------------
    // P enters as bf16 hi + lo parts (two products), so the probabilities
    // keep ~16 significant bits: the result matches fp32 P.V to rounding.
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      bf16x8 bp[NCT], bl[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const f32x4 a0 = S[2 * k2][ct];
        const f32x4 a1 = S[2 * k2 + 1][ct];
        const float v[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hw[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
          lw[i] = pack_bf16(v[2 * i] - __uint_as_float(hw[i] << 16), v[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u));
        }
        bp[ct] = __builtin_bit_cast(bf16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
        bl[ct] = __builtin_bit_cast(bf16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
      }
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const char* vp = st + vtr[d] + k2 * 8192;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp + 4096));
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          acc[d][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[ct], acc[d][ct], 0, 0, 0);
          acc[d][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[ct], acc[d][ct], 0, 0, 0);
        }
      }
    }

    // ---- end of this workgroup's part of the pair: write the partial record --
    if (s == w.nseg - 1 || g == g1 - 1) {
      const int pair = layer * p.hkv + h;
      float* rec = p.partial + (static_cast<int64_t>(pair) + blockIdx.x) * (16 * NCT) * kPartStride;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        float l = l_run[ct];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        float* row = rec + (16 * ct + ln) * kPartStride;
        if (lg == 0) {
          row[0] = m_run[ct];
          row[1] = l;
        }
#pragma unroll
        for (int d = 0; d < 2; ++d)
          *reinterpret_cast<f32x4*>(row + 2 + 16 * (2 * wave + d) + 4 * lg) = acc[d][ct];
      }
      reset();
    }
  };

  // every slot of an iteration runs its wait / barrier / copy, so that all
  // paths issue the same copies (the compiler's own waits stay exact)
  for (int g = g0; g < g1; g += kNS) {
    body(std::integral_constant<int, 0>{}, g);
    body(std::integral_constant<int, 1>{}, g + 1);
    body(std::integral_constant<int, 2>{}, g + 2);
    if (kNS > 3) body(std::integral_constant<int, (kNS > 3 ? 3 : 0)>{}, g + 3);
  }
  __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));   // the trailing empty copies retire before exit
}

// Combines the partial records of every pair: one workgroup per (pair, row),
// one thread per output dim.  Workgroup i wrote slot pair + i for each pair
// its tile range touched; the ranges of a pair's first and last tiles give
// the workgroups.  Runs after the streaming kernel on the same stream.
__global__ __launch_bounds__(kHeadDim) void attend_stream_merge(const AttendParams p, const StreamWork w,
                                                                int ncol_rows) {
  const int pair = blockIdx.x;
  const int row = blockIdx.y;
  const int d = threadIdx.x;
  if (row >= w.rows) return;
  // workgroup holding tile x: the largest i with i T / W <= x
  auto wg_of = [&](int64_t x) {
    const int64_t i = ((x + 1) * w.nwg - 1) / w.total;
    return static_cast<int>(min(i, static_cast<int64_t>(w.nwg - 1)));
  };
  const int64_t x0 = static_cast<int64_t>(pair) * w.nseg;
  const int i0 = wg_of(x0);
  const int i1 = wg_of(x0 + w.nseg - 1);
  float mt = -INFINITY;
  for (int i = i0; i <= i1; ++i)
    mt = fmaxf(mt, p.partial[((static_cast<int64_t>(pair) + i) * ncol_rows + row) * kPartStride]);
  float L = 0.0f, A = 0.0f;
  for (int i = i0; i <= i1; ++i) {
    const float* r = p.partial + ((static_cast<int64_t>(pair) + i) * ncol_rows + row) * kPartStride;
    const float sw = (r[0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(r[0] - mt);
    L += r[1] * sw;
    A += r[2 + d] * sw;
  }
  const int layer = pair / p.hkv;
  const int h = pair - layer * p.hkv;
  // decode's append: the new token (chunk token 0) also goes into the freed
  // ring slot, which the streaming kernel did not read
  if (p.write_slot >= 0 && row == 0) {
    const int64_t so = p.kv_ls * layer + static_cast<int64_t>(h) * kHeadDim + d;
    const int64_t dof = p.rec_ls * layer + (static_cast<int64_t>(h) * p.R + p.write_slot) * kHeadDim + d;
    p.rec_k[dof] = p.k_new[so];
    p.rec_v[dof] = p.v_new[so];
  }
  const int t = row / p.G;
  const int hh = h * p.G + row % p.G;
  const int hq = p.hkv * p.G;
  p.out[p.q_ls * layer + (static_cast<int64_t>(t) * hq + hh) * kHeadDim + d] = f32_to_bf16(A / L);
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

template <int NCT>
int launch_ncT(const AttendParams& p, const StreamWork& w, hipStream_t s) {
  hipLaunchKernelGGL(attend_stream_kernel<NCT>, dim3(w.nwg), dim3(kDcThreads), 0, s, p, w);
  hipLaunchKernelGGL(attend_stream_merge, dim3(w.npair, 16 * NCT), dim3(kHeadDim), 0, s, p, w, 16 * NCT);
  return 0;
}

}  // namespace

int stream_workgroups(int num_layers, int num_kv_heads) {
  const int cus = device_cus();
  if (cus <= 0) return 0;
  const int npair = num_layers * num_kv_heads;
  // at most ~4 pairs per workgroup range; never more than kMaxStreamWorkgroups
  int nwg = cus;
  while (nwg < npair / 4 && nwg * 2 <= kMaxStreamWorkgroups) nwg *= 2;
  return nwg < kMaxStreamWorkgroups ? nwg : kMaxStreamWorkgroups;
}

int launch_attend_stream(const AttendParams& p, int num_layers, hipStream_t s) {
  const int rows = p.tq * p.G;
  if (rows > 32 || p.allowed != nullptr || p.partial == nullptr || p.splits != 1) return -1;
  StreamWork w;
  w.npair = num_layers * p.hkv;
  w.nseg = p.nseg;
  const int64_t total = static_cast<int64_t>(w.npair) * w.nseg;
  if (total >= (int64_t{1} << 31)) return -1;
  w.total = static_cast<int>(total);
  w.rows = rows;
  w.nwg = stream_workgroups(num_layers, p.hkv);
  if (w.nwg <= 0) return -1;
  if (w.nwg > w.total) w.nwg = w.total;
  if ((w.total + w.nwg - 1) / w.nwg >= kIdsMax) return -1;   // a range's block ids must fit LDS
  return rows <= 16 ? launch_ncT<1>(p, w, s) : launch_ncT<2>(p, w, s);
}

}  // namespace nkv
