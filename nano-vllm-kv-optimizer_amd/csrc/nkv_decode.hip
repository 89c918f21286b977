// Streaming few-query attention (the decode layer-step's gather + attention)
// on gfx950: a persistent, stream-K kernel that keeps HBM busy.
//
// The work is the flat list of (pair, segment) tiles, pair = (layer, KV
// head), segments as in nkv_attend.hip (selected history blocks read in
// place, sink, physical ring pieces masked to the logical window, the causal
// chunk).  Every wavefront of the grid takes a contiguous range of the
// T = pairs x segments tiles, so all wavefronts stream the same number of
// bytes whatever the layer / head boundaries.
//
// A wavefront runs alone on its SIMD (all 512 registers) and keeps two tiles
// of K and V in flight in registers while it computes a third: a loaded HBM
// latency of several microseconds needs well over 128 KiB in flight per CU,
// more than the LDS holds.  Loads go through bounds-checked buffer
// descriptors (rows past a segment read as zero, no index clamping); slots
// past the range issue the same loads with an empty descriptor, so every path
// through the loop has the same loads and the compiler's waits stay exact.
//
// Per tile: S^T = K . Q^T on the matrix cores (A = 16 keys x 32 dims straight
// from the loaded registers, B = the pair's query rows from LDS), fp32 online
// softmax, O^T += V^T . P^T on the matrix cores too: the wave writes its V
// tile to its own LDS area and reads it back transposed (ds_read_b64_tr_b16);
// P enters as bf16 hi + lo parts, so P.V keeps fp32 accuracy.  At the end of its part of a pair a wavefront writes a partial
// (m, l, acc) record, slot pair + wavefront index; attend_stream_merge
// combines the records of each pair.
#include <type_traits>

#include "nkv_stage.h"

namespace nkv {
namespace {
using namespace attend_detail;
using namespace stage;

#ifndef NKV_DECODE_DEPTH
#define NKV_DECODE_DEPTH 1   // tiles in flight per wavefront beyond the one computed
#endif

constexpr int kDcThreads = 256;
constexpr int kIdsMax = 512;      // tiles per workgroup range (block ids staged in LDS)
constexpr int kQPairs = 8;        // pairs per workgroup range (query rows staged in LDS)

struct StreamWork {
  int total;       // pairs x segments (< 2^31, checked by the launcher)
  int npair;
  int nseg;
  int nwg;         // workgroups
  int nwave;       // wavefronts = partition units
  int rows;        // query rows of a pair (tq x G), <= 4
};

// K / V of one tile in registers: lane (lg, ln) holds
//   k[i][s] = dims 32 s + 8 lg .. +8 of key 16 i + ln   (the MFMA A operand)
//   v[j]    = dims 8 ln .. +8 of key 4 j + lg            (written to LDS for P.V)
struct TileRegs {
  u32x4 k[4][4];
  u32x4 v[16];
};

template <int M>
__global__ __launch_bounds__(kDcThreads, 1) void attend_wave_kernel(const AttendParams p, const StreamWork w) {
  __shared__ int ids_lds[kIdsMax];
  __shared__ __attribute__((aligned(16))) char q_lds[kQPairs * 16 * 256];
  __shared__ __attribute__((aligned(16))) char v_lds[4][kTileBytes];   // per-wave V tile (stage.h V layout)

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int ln = lane & 15;
  const int lg = lane >> 4;
  const int hq = p.hkv * p.G;
  const int wg0 = static_cast<int>(static_cast<int64_t>(blockIdx.x) * w.total / w.nwg);
  const int wg1 = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * w.total / w.nwg);
  const int gw = blockIdx.x * 4 + wave;
  const int t0 = static_cast<int>(static_cast<int64_t>(gw) * w.total / w.nwave);
  const int t1 = static_cast<int>(static_cast<int64_t>(gw + 1) * w.total / w.nwave);
  const int pair_lo = wg0 / w.nseg;

  // ---- stage the workgroup's block ids and query rows in LDS ----------------
  for (int i = tid; i < wg1 - wg0; i += kDcThreads) {
    const int g = wg0 + i;
    const int pair = g / w.nseg;
    const int sg = g - pair * w.nseg;
    const int layer = pair / p.hkv;
    ids_lds[i] = sg < p.n_hist ? p.ids[static_cast<int64_t>(layer) * p.ids_ls + sg] : 0;
  }
  if (wg1 > wg0) {
    const int npl = (wg1 - 1) / w.nseg - pair_lo + 1;   // <= kQPairs (checked by the launcher)
    for (int i = tid; i < npl * 16 * 16; i += kDcThreads) {
      const int pl = i >> 8;
      const int row = (i >> 4) & 15;
      const int c = i & 15;
      const int pair = pair_lo + pl;
      const int layer = pair / p.hkv;
      const int h = pair - layer * p.hkv;
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (row < w.rows) {
        const int t = row / p.G;
        const int hh = h * p.G + row % p.G;
        v = *reinterpret_cast<const u32x4*>(p.q + p.q_ls * layer + (static_cast<int64_t>(t) * hq + hh) * kHeadDim + c * 8);
      }
      // row-swizzled chunks: the B-operand reads (16 rows, one chunk) hit all banks
      *reinterpret_cast<u32x4*>(q_lds + (pl * 16 + row) * 256 + ((c ^ row) << 4)) = v;
    }
  }
  __syncthreads();
  if (t0 >= t1) return;

  // tile index -> (layer, KV head, segment); uniform, in scalar registers
  auto seg_of = [&](int g, int* layer, int* h, int* s) __attribute__((always_inline)) {
    const int pair = __builtin_amdgcn_readfirstlane(g / w.nseg);
    *s = __builtin_amdgcn_readfirstlane(g - pair * w.nseg);
    *layer = __builtin_amdgcn_readfirstlane(pair / p.hkv);
    *h = __builtin_amdgcn_readfirstlane(pair - *layer * p.hkv);
  };
  auto seg_at = [&](int g, int layer, int h, int s) __attribute__((always_inline)) {
    return make_seg_blk<NKV_KV_BF16>(p, layer, h, s, __builtin_amdgcn_readfirstlane(ids_lds[g - wg0]));
  };
  // Every slot loads, also past the range: a slot past it reads the first
  // 256 bytes of q over and over (cache-resident, no HBM traffic), so that
  // every path through the loop issues the same loads.  Rows past a segment
  // are clamped to its last row (masked below).
  auto load = [&](int g, TileRegs& r) __attribute__((always_inline)) {
    const bool live = g < t1;
    const int gc = live ? g : t1 - 1;
    int layer, h, s;
    seg_of(gc, &layer, &h, &s);
    const Seg sg = seg_at(gc, layer, h, s);
    const char* kb = live ? sg.kbase : reinterpret_cast<const char*>(p.q);
    const char* vb = live ? sg.vbase : reinterpret_cast<const char*>(p.q);
    const int rowb = live ? sg.rowb : 0;
    const int last = live ? sg.len - 1 : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const char* rp = kb + min(16 * i + ln, last) * rowb + 16 * lg;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) r.k[i][s4] = *reinterpret_cast<const u32x4*>(rp + 64 * s4);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
      r.v[j] = *reinterpret_cast<const u32x4*>(vb + min(4 * j + lg, last) * rowb + 16 * ln);
  };

  float m_run = -INFINITY;   // per query row (lane & 15)
  float l_run = 0.0f;        // partial over this lane group's keys
  f32x4 acc[8];              // O^T: acc[dt][i] = dim 16 dt + 4 lg + i of query row ln
  auto reset = [&]() __attribute__((always_inline)) {
    m_run = -INFINITY;
    l_run = 0.0f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  };
  reset();
  char* my_v = v_lds[wave];
  // V register (key 4 j + lg, chunk ln) -> its swizzled LDS position
  const int vw = lg * 256 + ((ln ^ (2 * lg)) << 4);
  // transposing V read for dims 16 dt + ..: lane ln addresses key 4 lg + (ln >> 2)
  // (+ 32 k2 + 16 half), dims 16 dt + 4 (ln & 3); dt & 4 -> + 128, dt & 3 picks vtr[]
  int vtr[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    vtr[q] = (4 * lg + (ln >> 2)) * 256 + ((2 * (q ^ (ln >> 2)) + ((ln & 3) >> 1)) << 4) + 8 * (ln & 1);

  auto compute = [&](int g, const TileRegs& r) __attribute__((always_inline)) {
    if (g >= t1) return;
    int layer, h, s;
    seg_of(g, &layer, &h, &s);
    const Seg cur = seg_at(g, layer, h, s);
    const char* qa = q_lds + (layer * p.hkv + h - pair_lo) * 16 * 256;

    // V tile -> this wave's LDS area (key-major, swizzled) for the transposing reads
#pragma unroll
    for (int j = 0; j < 16; ++j) *reinterpret_cast<u32x4*>(my_v + j * 1024 + vw) = r.v[j];

    // ---- S^T = K . Q^T: c[i][e] = key 16 i + 4 lg + e, query row ln ----------
    f32x4 c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const bf16x8 bq = *reinterpret_cast<const bf16x8*>(qa + ln * 256 + (((4 * s4 + lg) ^ ln) << 4));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        c[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.k[i][s4]), bq, c[i], 0, 0, 0);
    }

    // ---- visibility ----------------------------------------------------------
    const bool full = cur.type == kSegHist ? cur.vlen == kBlock
                    : cur.type == kSegSink ? cur.len == kBlock
                    : cur.type == kSegRecent ? (p.rec_len == p.R && cur.len == kBlock)
                    : false;
    if (!full) {
      if (cur.type == kSegRecent) {
        int a = (cur.off - p.ring_base - p.rec_lo) % p.R;
        a = a < 0 ? a + p.R : a;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = 16 * i + 4 * lg + e;
            int x = a + key;
            x -= p.R & ((p.R - 1 - x) >> 31);
            c[i][e] = fminf(c[i][e], vis_bound(max(key - (cur.vlen - 1), x - (p.rec_len - 1))));
          }
      } else {
        int thr = cur.vlen - 1;
        if (cur.type == kSegChunk) thr = min(thr, ln / p.G - cur.off);
        const int base = 4 * lg - thr;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) c[i][e] = fminf(c[i][e], vis_bound(base + 16 * i + e));
      }
    }

    // ---- online softmax (fp32, lazy reference max) ---------------------------
    float cmax = c[0][0];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) cmax = fmaxf(cmax, c[i][e]);
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
    const float cand = cmax * p.scale_log2;
    const float m_new = cand > m_run + 8.0f ? cand : m_run;
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c[i][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(c[i][e], p.scale_log2, -m_use));
        lsum += c[i][e];
      }
    l_run = l_run * alpha + lsum;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
    wave_lds_sync();   // the V tile is in LDS

    // ---- O^T += V^T . P^T on the matrix cores; P as bf16 hi + lo parts so the
    // probabilities keep ~16 significant bits (fp32-accurate P.V) ------------
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const float v8[8] = {c[2 * k2][0], c[2 * k2][1], c[2 * k2][2], c[2 * k2][3],
                           c[2 * k2 + 1][0], c[2 * k2 + 1][1], c[2 * k2 + 1][2], c[2 * k2 + 1][3]};
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hw[i] = pack_bf16(v8[2 * i], v8[2 * i + 1]);
        lw[i] = pack_bf16(v8[2 * i] - __uint_as_float(hw[i] << 16), v8[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u));
      }
      const bf16x8 bp = __builtin_bit_cast(bf16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
      const bf16x8 bl = __builtin_bit_cast(bf16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const char* vp = my_v + vtr[dt & 3] + (dt >> 2) * 128 + k2 * 8192;
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(vp + 4096));
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp, acc[dt], 0, 0, 0);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, acc[dt], 0, 0, 0);
      }
    }
    wave_lds_sync();   // the next tile may overwrite the V area

    // ---- end of this wavefront's part of the pair: write the partial record --
    if (s == w.nseg - 1 || g == t1 - 1) {
      float l = l_run;
      l += __shfl_xor(l, 16);
      l += __shfl_xor(l, 32);
      const int pair = layer * p.hkv + h;
      float* row = p.partial + ((static_cast<int64_t>(pair) + gw) * kMaxRows + ln) * kPartStride;
      if (lg == 0) {
        row[0] = m_run;
        row[1] = l;
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(row + 2 + 16 * dt + 4 * lg) = acc[dt];
      reset();
    }
  };

#if NKV_DECODE_DEPTH == 2
  // three register buffers: two tiles in flight while one is computed
  TileRegs b0, b1, b2;
  load(t0, b0);
  load(t0 + 1, b1);
  for (int g = t0; g < t1; g += 3) {
    load(g + 2, b2);
    compute(g, b0);
    load(g + 3, b0);
    compute(g + 1, b1);
    load(g + 4, b1);
    compute(g + 2, b2);
  }
#else
  // two register buffers: the next tile in flight while one is computed
  TileRegs b0, b1;
  load(t0, b0);
  for (int g = t0; g < t1; g += 2) {
    load(g + 1, b1);
    compute(g, b0);
    load(g + 2, b0);
    compute(g + 1, b1);
  }
#endif
}

// Combines the partial records of every pair: one workgroup per (pair, row),
// one thread per output dim.  Partition unit i (of w.nwave) wrote slot
// pair + i for each pair its tile range touched; the units holding the pair's
// first and last tiles bound them.  Runs after the streaming kernel on the
// same stream; also performs decode's append of the new token to the ring.
__global__ __launch_bounds__(kHeadDim) void attend_stream_merge(const AttendParams p, const StreamWork w) {
  const int pair = blockIdx.x;
  const int row = blockIdx.y;
  const int d = threadIdx.x;
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
  if (row >= w.rows) return;
  // partition unit holding tile x: the largest i with i T / N <= x
  auto unit_of = [&](int64_t x) {
    const int64_t i = ((x + 1) * w.nwave - 1) / w.total;
    return static_cast<int>(min(i, static_cast<int64_t>(w.nwave - 1)));
  };
  // units whose range is empty (more units than tiles) wrote nothing
  auto owns_tiles = [&](int i) {
    return static_cast<int64_t>(i) * w.total / w.nwave < static_cast<int64_t>(i + 1) * w.total / w.nwave;
  };
  const int64_t x0 = static_cast<int64_t>(pair) * w.nseg;
  const int i0 = unit_of(x0);
  const int i1 = unit_of(x0 + w.nseg - 1);
  float mt = -INFINITY;
  for (int i = i0; i <= i1; ++i)
    if (owns_tiles(i)) mt = fmaxf(mt, p.partial[((static_cast<int64_t>(pair) + i) * kMaxRows + row) * kPartStride]);
  float L = 0.0f, A = 0.0f;
  for (int i = i0; i <= i1; ++i) {
    if (!owns_tiles(i)) continue;
    const float* r = p.partial + ((static_cast<int64_t>(pair) + i) * kMaxRows + row) * kPartStride;
    const float sw = (r[0] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(r[0] - mt);
    L += r[1] * sw;
    A += r[2 + d] * sw;
  }
  const int t = row / p.G;
  const int hh = h * p.G + row % p.G;
  const int hq = p.hkv * p.G;
  p.out[p.q_ls * layer + (static_cast<int64_t>(t) * hq + hh) * kHeadDim + d] = f32_to_bf16(A / L);
}

template <int M>
void launch_m(const AttendParams& p, const StreamWork& w, hipStream_t s) {
  hipLaunchKernelGGL(attend_wave_kernel<M>, dim3(w.nwg), dim3(kDcThreads), 0, s, p, w);
  hipLaunchKernelGGL(attend_stream_merge, dim3(w.npair, kMaxRows), dim3(kHeadDim), 0, s, p, w);
}

}  // namespace

int stream_workgroups(int num_layers, int num_kv_heads) {
  const int cus = device_cus();
  if (cus <= 0) return 0;
  const int npair = num_layers * num_kv_heads;
  // one 4-wavefront workgroup per CU; more when pairs are many, so that a
  // workgroup range spans few pairs
  int nwg = cus;
  while (nwg < npair / 2 && nwg * 2 <= kMaxStreamWorkgroups) nwg *= 2;
  return nwg < kMaxStreamWorkgroups ? nwg : kMaxStreamWorkgroups;
}

int launch_attend_stream(const AttendParams& p, int num_layers, hipStream_t s) {
  // up to 4 query rows (decode: one token x G <= 4 heads): three K/V tile
  // buffers fit the register file only with the 4-row accumulator
  const int rows = p.tq * p.G;
  if (rows > 4 || p.allowed != nullptr || p.partial == nullptr) return -1;
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
  w.nwave = 4 * w.nwg;
  const int range = (w.total + w.nwg - 1) / w.nwg;
  if (range >= kIdsMax) return -1;                              // a range's block ids must fit LDS
  if ((range + w.nseg - 1) / w.nseg + 1 > kQPairs) return -1;  // and its pairs' query rows
  launch_m<4>(p, w, s);
  return 0;
}

}  // namespace nkv
