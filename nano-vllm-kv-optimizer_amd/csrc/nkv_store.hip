// HBM store maintenance: appending prefill chunks to the history (with the
// int8 schemes), building block representatives, updating the recent window
// and computing prefill query summaries.  These run once per prefill chunk
// (or verify commit), not per decode step.
#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kStoreThreads = 256;

// ---------------------------------------------------------------------------
// int8 K scale from the first chunk: m12_runtime.py:463-467
//   k_scale[h][d] = max(amax_t |k[t][h][d]|, 1e-8) / 127
// Pass 1 folds |k| into the (zeroed) k_scale buffer with an integer atomicMax
// on the fp32 bit pattern (monotone for non-negative floats); pass 2 turns the
// maxima into scales.
// ---------------------------------------------------------------------------
__global__ void fill_zero_kernel(float* __restrict__ x, int64_t n) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    x[i] = 0.0f;
}

__global__ __launch_bounds__(kHeadDim) void k_amax_kernel(const uint16_t* __restrict__ k,
                                                          int64_t kv_ls, int T, int hkv,
                                                          float* __restrict__ k_scale) {
  const int t0 = blockIdx.x * 64;
  const int h = blockIdx.y;
  const int layer = blockIdx.z;
  const int d = threadIdx.x;
  const uint16_t* kl = k + kv_ls * layer;
  float m = 0.0f;
  const int t1 = min(T, t0 + 64);
  for (int t = t0; t < t1; ++t)
    m = fmaxf(m, fabsf(bf16_to_f32(kl[(static_cast<int64_t>(t) * hkv + h) * kHeadDim + d])));
  atomicMax(reinterpret_cast<unsigned int*>(&k_scale[(static_cast<int64_t>(layer) * hkv + h) * kHeadDim + d]),
            __float_as_uint(m));
}

__global__ void k_scale_finalize_kernel(float* __restrict__ k_scale, int64_t n) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i < n) k_scale[i] = fmaxf(k_scale[i], 1e-8f) / 127.0f;
}

// ---------------------------------------------------------------------------
// History append: one workgroup per (block, KV head, layer).  Thread t owns
// token t/4 of the block and 32 dims (t%4)*32 .. +32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int8_t q8(float x, float s) {
  float r = rintf(x / s);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return static_cast<int8_t>(static_cast<int>(r));
}

__global__ __launch_bounds__(kStoreThreads) void store_chunk_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t kv_ls, int T,
    int start_block, int hkv, int cap, int fmt, void* __restrict__ hist_k,
    void* __restrict__ hist_v, int64_t hist_ls, const float* __restrict__ k_scale,
    float* __restrict__ v_scale, uint16_t* __restrict__ k_tscale, uint16_t* __restrict__ v_tscale,
    uint16_t* __restrict__ sink_k, uint16_t* __restrict__ sink_v, int64_t sink_ls, int S,
    int sink_write_len) {
  __shared__ float s_red[kStoreThreads / kWave];
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int layer = blockIdx.z;
  const int tid = threadIdx.x;
  const int tl = tid >> 2;          // token in block
  const int d0 = (tid & 3) * 32;    // first dim
  const int t = b * kBlock + tl;    // token in chunk
  const bool valid = t < T;

  float kf[32], vf[32];
  {
    const uint4* ks = reinterpret_cast<const uint4*>(k + kv_ls * layer + (static_cast<int64_t>(t) * hkv + h) * kHeadDim + d0);
    const uint4* vs = reinterpret_cast<const uint4*>(v + kv_ls * layer + (static_cast<int64_t>(t) * hkv + h) * kHeadDim + d0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 a = valid ? ks[c] : make_uint4(0u, 0u, 0u, 0u);
      const uint4 bb = valid ? vs[c] : make_uint4(0u, 0u, 0u, 0u);
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
      const uint32_t bw[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kf[c * 8 + 2 * i] = bf16_lo(aw[i]);
        kf[c * 8 + 2 * i + 1] = bf16_hi(aw[i]);
        vf[c * 8 + 2 * i] = bf16_lo(bw[i]);
        vf[c * 8 + 2 * i + 1] = bf16_hi(bw[i]);
      }
    }
  }

  // sink: the first min(S, T) tokens of the first chunk (m12_runtime.py:482-486)
  if (t < sink_write_len) {
    uint4* sk = reinterpret_cast<uint4*>(sink_k + sink_ls * layer + (static_cast<int64_t>(h) * S + t) * kHeadDim + d0);
    uint4* sv = reinterpret_cast<uint4*>(sink_v + sink_ls * layer + (static_cast<int64_t>(h) * S + t) * kHeadDim + d0);
    const uint4* ks = reinterpret_cast<const uint4*>(k + kv_ls * layer + (static_cast<int64_t>(t) * hkv + h) * kHeadDim + d0);
    const uint4* vs = reinterpret_cast<const uint4*>(v + kv_ls * layer + (static_cast<int64_t>(t) * hkv + h) * kHeadDim + d0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      sk[c] = ks[c];
      sv[c] = vs[c];
    }
  }

  const int blk = start_block + b;
  const int64_t row = hist_ls * layer + ((static_cast<int64_t>(h) * cap + blk) * kBlock + tl) * kHeadDim + d0;
  if (fmt == NKV_KV_BF16) {
    uint4* dk = reinterpret_cast<uint4*>(static_cast<uint16_t*>(hist_k) + row);
    uint4* dv = reinterpret_cast<uint4*>(static_cast<uint16_t*>(hist_v) + row);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t ow[4], pw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ow[i] = (__float_as_uint(kf[c * 8 + 2 * i]) >> 16) | (__float_as_uint(kf[c * 8 + 2 * i + 1]) & 0xffff0000u);
        pw[i] = (__float_as_uint(vf[c * 8 + 2 * i]) >> 16) | (__float_as_uint(vf[c * 8 + 2 * i + 1]) & 0xffff0000u);
      }
      dk[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      dv[c] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    }
    return;
  }

  float kscale[32], vscale_tok = 1.0f, kscale_tok = 1.0f, vs_blk = 1.0f;
  if (fmt == NKV_KV_INT8_CHANNEL) {
    const float* ks = k_scale + (static_cast<int64_t>(layer) * hkv + h) * kHeadDim + d0;
#pragma unroll
    for (int i = 0; i < 32; ++i) kscale[i] = ks[i];
    // V: per-(block, head) scale over all 64 x 128 values (m12_runtime.py:469-474)
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) am = fmaxf(am, fabsf(vf[i]));
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    if ((tid & 63) == 0) s_red[tid >> 6] = am;
    __syncthreads();
    am = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    vs_blk = fmaxf(am, 1e-8f) / 127.0f;
    if (tid == 0) v_scale[(static_cast<int64_t>(layer) * hkv + h) * cap + blk] = vs_blk;
  } else {
    // per-token fp16 scales: s = fp16(max(amax_d |x| / 127, 2^-24))
    float ak = 0.0f, av = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      ak = fmaxf(ak, fabsf(kf[i]));
      av = fmaxf(av, fabsf(vf[i]));
    }
    ak = fmaxf(ak, __shfl_xor(ak, 1));
    ak = fmaxf(ak, __shfl_xor(ak, 2));
    av = fmaxf(av, __shfl_xor(av, 1));
    av = fmaxf(av, __shfl_xor(av, 2));
    const __half hk = __float2half_rn(fmaxf(ak / 127.0f, 5.9604644775390625e-08f));
    const __half hv = __float2half_rn(fmaxf(av / 127.0f, 5.9604644775390625e-08f));
    kscale_tok = __half2float(hk);
    vscale_tok = __half2float(hv);
    if ((tid & 3) == 0) {
      const int64_t ti = (static_cast<int64_t>(layer) * hkv + h) * cap * kBlock + static_cast<int64_t>(blk) * kBlock + tl;
      k_tscale[ti] = __half_as_ushort(hk);
      v_tscale[ti] = __half_as_ushort(hv);
    }
  }
  int8_t* dk = static_cast<int8_t*>(hist_k) + row;
  int8_t* dv = static_cast<int8_t*>(hist_v) + row;
  uint32_t kw[8], vw[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t a = 0u, c = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = w * 4 + i;
      const float sk = (fmt == NKV_KV_INT8_CHANNEL) ? kscale[idx] : kscale_tok;
      const float sv = (fmt == NKV_KV_INT8_CHANNEL) ? vs_blk : vscale_tok;
      a |= (static_cast<uint32_t>(static_cast<uint8_t>(q8(kf[idx], sk)))) << (8 * i);
      c |= (static_cast<uint32_t>(static_cast<uint8_t>(q8(vf[idx], sv)))) << (8 * i);
    }
    kw[w] = a;
    vw[w] = c;
  }
  reinterpret_cast<uint4*>(dk)[0] = make_uint4(kw[0], kw[1], kw[2], kw[3]);
  reinterpret_cast<uint4*>(dk)[1] = make_uint4(kw[4], kw[5], kw[6], kw[7]);
  reinterpret_cast<uint4*>(dv)[0] = make_uint4(vw[0], vw[1], vw[2], vw[3]);
  reinterpret_cast<uint4*>(dv)[1] = make_uint4(vw[4], vw[5], vw[6], vw[7]);
}

// ---------------------------------------------------------------------------
// Representatives: one wavefront per (block, KV head, layer); lane = token.
// m12_runtime.py:354-395.
// ---------------------------------------------------------------------------
constexpr int kDirPad = kHeadDim + 1;

__global__ __launch_bounds__(kWave) void build_reps_kernel(
    const uint16_t* __restrict__ k, int64_t kv_ls, int T, int start_block, int hkv, int cap,
    int r, uint16_t* __restrict__ reps, int64_t reps_ls) {
  __shared__ float s_dir[kBlock * kDirPad];
  __shared__ float s_mean[kHeadDim];
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int layer = blockIdx.z;
  const int lane = threadIdx.x;
  const int t = b * kBlock + lane;
  const bool valid = t < T;
  const uint16_t* kl = k + kv_ls * layer;

  // normalise this lane's key (F.normalize: x / max(||x||, 1e-12))
  float x[kHeadDim];
  {
    const uint4* src = reinterpret_cast<const uint4*>(kl + (static_cast<int64_t>(t) * hkv + h) * kHeadDim);
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const uint4 a = valid ? src[c] : make_uint4(0u, 0u, 0u, 0u);
      x[c * 8 + 0] = bf16_lo(a.x); x[c * 8 + 1] = bf16_hi(a.x);
      x[c * 8 + 2] = bf16_lo(a.y); x[c * 8 + 3] = bf16_hi(a.y);
      x[c * 8 + 4] = bf16_lo(a.z); x[c * 8 + 5] = bf16_hi(a.z);
      x[c * 8 + 6] = bf16_lo(a.w); x[c * 8 + 7] = bf16_hi(a.w);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int d = 0; d < kHeadDim; ++d) ss = __builtin_fmaf(x[d], x[d], ss);
  const float den = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
  for (int d = 0; d < kHeadDim; ++d) {
    x[d] = x[d] / den;
    s_dir[lane * kDirPad + d] = x[d];
  }
  __syncthreads();

  // mean direction over the block's tokens
  float m0 = 0.0f, m1 = 0.0f;
  for (int tt = 0; tt < kBlock; ++tt) {
    m0 += s_dir[tt * kDirPad + lane];
    m1 += s_dir[tt * kDirPad + lane + 64];
  }
  m0 *= (1.0f / kBlock);
  m1 *= (1.0f / kBlock);
  float mss = m0 * m0 + m1 * m1;
  for (int o = 32; o > 0; o >>= 1) mss += __shfl_xor(mss, o);
  const float mden = fmaxf(sqrtf(mss), 1e-12f);
  s_mean[lane] = m0 / mden;
  s_mean[lane + 64] = m1 / mden;
  __syncthreads();

  // seed: first argmax of cos to the mean direction
  float cs = 0.0f;
#pragma unroll
  for (int d = 0; d < kHeadDim; ++d) cs = __builtin_fmaf(x[d], s_mean[d], cs);
  float bv = cs;
  int bi = lane;
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  // raw bf16 row of each chosen token -> reps[h][start_block + b][j][:]
  uint16_t* dst = reps + reps_ls * layer + ((static_cast<int64_t>(h) * cap + start_block + b) * r) * kHeadDim;
  auto write_rep = [&](int j, int tok) {
    const int tt = b * kBlock + tok;
    if (lane < 16) {
      uint4 a = make_uint4(0u, 0u, 0u, 0u);
      if (tt < T) a = reinterpret_cast<const uint4*>(kl + (static_cast<int64_t>(tt) * hkv + h) * kHeadDim)[lane];
      reinterpret_cast<uint4*>(dst + static_cast<int64_t>(j) * kHeadDim)[lane] = a;
    }
  };
  write_rep(0, bi);
  int last = bi;
  bool is_chosen = (lane == bi);
  float maxcos = -INFINITY;
  for (int step = 1; step < r; ++step) {
    float c = 0.0f;
#pragma unroll
    for (int d = 0; d < kHeadDim; ++d) c = __builtin_fmaf(x[d], s_dir[last * kDirPad + d], c);
    maxcos = fmaxf(maxcos, c);
    float val = is_chosen ? fmaxf(maxcos, 2.0f) : maxcos;
    int vi = lane;
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(val, o);
      const int oi = __shfl_xor(vi, o);
      if (ov < val || (ov == val && oi < vi)) {
        val = ov;
        vi = oi;
      }
    }
    write_rep(step, vi);
    last = vi;
    is_chosen = is_chosen || (lane == vi);
  }
}

// ---------------------------------------------------------------------------
// Recent window on the logical buffer (one workgroup per KV head and layer).
// Carry moves logical [X, X + carry) -> [0, carry) with X = old_len - carry
// >= 0, processed in ascending 64-token chunks with a barrier between each
// chunk's reads and writes: a chunk's writes land below every later chunk's
// sources, so the forward copy never reads a clobbered slot.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kStoreThreads) void recent_update_kernel(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t kv_ls, int src_lo,
    int n_src, int ring_start, int old_len, int carry, int hkv, int R,
    uint16_t* __restrict__ rk, uint16_t* __restrict__ rv, int64_t rec_ls) {
  const int h = blockIdx.x;
  const int layer = blockIdx.y;
  const int tid = threadIdx.x;
  const int tl = tid >> 2;
  const int c0 = (tid & 3) * 4;   // uint4 index in the 16-chunk row
  uint4* rkl = reinterpret_cast<uint4*>(rk + rec_ls * layer + static_cast<int64_t>(h) * R * kHeadDim);
  uint4* rvl = reinterpret_cast<uint4*>(rv + rec_ls * layer + static_cast<int64_t>(h) * R * kHeadDim);
  const int X = old_len - carry;
  for (int base = 0; base < carry; base += kBlock) {
    const int i = base + tl;
    uint4 a[4], bb[4];
    if (i < carry) {
      const int src = (ring_start + X + i) % R;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        a[c] = rkl[src * 16 + c0 + c];
        bb[c] = rvl[src * 16 + c0 + c];
      }
    }
    __syncthreads();
    if (i < carry) {
      const int dst = (ring_start + i) % R;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        rkl[dst * 16 + c0 + c] = a[c];
        rvl[dst * 16 + c0 + c] = bb[c];
      }
    }
    __syncthreads();
  }
  for (int i = tid >> 2; i < n_src; i += kStoreThreads / 4) {
    const int dst = (ring_start + carry + i) % R;
    const uint4* sk = reinterpret_cast<const uint4*>(k + kv_ls * layer + (static_cast<int64_t>(src_lo + i) * hkv + h) * kHeadDim);
    const uint4* sv = reinterpret_cast<const uint4*>(v + kv_ls * layer + (static_cast<int64_t>(src_lo + i) * hkv + h) * kHeadDim);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      rkl[dst * 16 + c0 + c] = sk[c0 + c];
      rvl[dst * 16 + c0 + c] = sv[c0 + c];
    }
  }
}

// ---------------------------------------------------------------------------
// Query summaries: bf16 RNE of the fp64 mean (prefill_query_summaries).
// The fp64 sum of bf16 values is exact at these lengths; the quotient is
// rounded to fp32 with round-to-odd and then to bf16 with RNE, which equals a
// single rounding of the fp64 quotient to bf16.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint16_t f64_to_bf16(double x) {
  float f = __double2float_rz(x);
  if (static_cast<double>(f) != x && isfinite(f)) f = __uint_as_float(__float_as_uint(f) | 1u);
  return f32_to_bf16(f);
}

__global__ __launch_bounds__(kStoreThreads) void query_mean_kernel(
    const uint16_t* __restrict__ q, int64_t q_ls, int T, int nelem, int nseg,
    uint16_t* __restrict__ out, int64_t out_ls) {
  const int e = blockIdx.x * kStoreThreads + threadIdx.x;
  const int s = blockIdx.y;
  const int layer = blockIdx.z;
  if (e >= nelem) return;
  const int base = T / nseg, extra = T % nseg;
  const int lo = s * base + min(s, extra);
  const int hi = lo + base + (s < extra ? 1 : 0);
  const uint16_t* ql = q + q_ls * layer;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  int t = lo;
  for (; t + 3 < hi; t += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += static_cast<double>(bf16_to_f32(ql[static_cast<int64_t>(t + u) * nelem + e]));
  }
  for (; t < hi; ++t) acc[0] += static_cast<double>(bf16_to_f32(ql[static_cast<int64_t>(t) * nelem + e]));
  const double sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  out[out_ls * layer + static_cast<int64_t>(s) * nelem + e] = f64_to_bf16(sum / static_cast<double>(hi - lo));
}

// The same means with 16-byte loads: a workgroup owns 16 chunks of 8
// elements and splits the segment's tokens over 16 thread groups, each with 8
// rows in flight; the groups' fp64 partial sums meet in LDS.  The sums are
// exact in fp64 (bf16 values of any realistic exponent spread), so the result
// does not depend on the order and equals query_mean_kernel's.
constexpr int kQmChunks = 16;
constexpr int kQmGroups = kStoreThreads / kQmChunks;
constexpr int kQmUnroll = 8;
__global__ __launch_bounds__(kStoreThreads) void query_mean8_kernel(
    const uint16_t* __restrict__ q, int64_t q_ls, int T, int nelem, int nseg,
    uint16_t* __restrict__ out, int64_t out_ls) {
  __shared__ double s_part[kQmGroups][kQmChunks * 8];
  const int cl = threadIdx.x % kQmChunks;
  const int grp = threadIdx.x / kQmChunks;
  const int nc = nelem >> 3;
  const int c = blockIdx.x * kQmChunks + cl;
  const int s = blockIdx.y;
  const int layer = blockIdx.z;
  const int base = T / nseg, extra = T % nseg;
  const int lo = s * base + min(s, extra);
  const int hi = lo + base + (s < extra ? 1 : 0);
  double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  auto add = [&](const uint4& v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += static_cast<double>(bf16_lo(w[i]));
      acc[2 * i + 1] += static_cast<double>(bf16_hi(w[i]));
    }
  };
  if (c < nc) {
    const uint4* ql = reinterpret_cast<const uint4*>(q + q_ls * layer);
    int t = lo + grp;
    for (; t + (kQmUnroll - 1) * kQmGroups < hi; t += kQmUnroll * kQmGroups) {
      uint4 v[kQmUnroll];
#pragma unroll
      for (int u = 0; u < kQmUnroll; ++u) v[u] = ql[static_cast<int64_t>(t + u * kQmGroups) * nc + c];
#pragma unroll
      for (int u = 0; u < kQmUnroll; ++u) add(v[u]);
    }
    for (; t < hi; t += kQmGroups) add(ql[static_cast<int64_t>(t) * nc + c]);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_part[grp][cl * 8 + e] = acc[e];
  __syncthreads();
  if (threadIdx.x < kQmChunks * 8) {
    const int c2 = blockIdx.x * kQmChunks + threadIdx.x / 8;
    if (c2 < nc) {
      double sum = 0.0;
#pragma unroll
      for (int g = 0; g < kQmGroups; ++g) sum += s_part[g][threadIdx.x];
      out[out_ls * layer + static_cast<int64_t>(s) * nelem + c2 * 8 + threadIdx.x % 8] =
          f64_to_bf16(sum / static_cast<double>(hi - lo));
    }
  }
}

}  // namespace
}  // namespace nkv

using namespace nkv;

extern "C" int nkv_store_chunk(const nkv_store* st, int layer0, int num_layers, const uint16_t* k,
                               const uint16_t* v, int64_t kv_layer_stride, int T, int start_block,
                               int compute_k_scale, int write_sink, void* stream) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_ARG(k != nullptr && v != nullptr, "nkv_store_chunk: k and v must be non-NULL");
  NKV_CHECK_ARG(T >= 1, "nkv_store_chunk: T must be >= 1 (got %d)", T);
  const int nblk = (T + kBlock - 1) / kBlock;
  NKV_CHECK_ARG(start_block >= 0 && start_block + nblk <= st->cap_blocks,
                "nkv_store_chunk: blocks [%d, %d) exceed cap_blocks %d", start_block, start_block + nblk,
                st->cap_blocks);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int hkv = st->num_kv_heads;
  if (st->kv_format == NKV_KV_INT8_CHANNEL && compute_k_scale) {
    float* ks = st->k_scale + static_cast<int64_t>(layer0) * hkv * kHeadDim;
    const int64_t n = static_cast<int64_t>(num_layers) * hkv * kHeadDim;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, ks, n);
    hipLaunchKernelGGL(k_amax_kernel, dim3((T + 63) / 64, hkv, num_layers), dim3(kHeadDim), 0, s, k,
                       kv_layer_stride, T, hkv, ks);
    hipLaunchKernelGGL(k_scale_finalize_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, ks, n);
    rc = launch_status("nkv_store_chunk/k_scale");
    if (rc != NKV_OK) return rc;
  }
  const int64_t hist_ls = static_cast<int64_t>(hkv) * st->cap_blocks * kBlock * kHeadDim;
  const int64_t elem = st->kv_format == NKV_KV_BF16 ? 2 : 1;
  const int64_t sink_ls = static_cast<int64_t>(hkv) * st->sink_tokens * kHeadDim;
  const int64_t ts_ls = static_cast<int64_t>(hkv) * st->cap_blocks * kBlock;
  const int sink_write_len = (write_sink && st->sink_tokens > 0) ? (T < st->sink_tokens ? T : st->sink_tokens) : 0;
  hipLaunchKernelGGL(
      store_chunk_kernel, dim3(nblk, hkv, num_layers), dim3(kStoreThreads), 0, s, k, v, kv_layer_stride, T,
      start_block, hkv, st->cap_blocks, st->kv_format,
      static_cast<void*>(static_cast<char*>(st->hist_k) + layer0 * hist_ls * elem),
      static_cast<void*>(static_cast<char*>(st->hist_v) + layer0 * hist_ls * elem), hist_ls,
      st->k_scale ? st->k_scale + static_cast<int64_t>(layer0) * hkv * kHeadDim : nullptr,
      st->v_scale ? st->v_scale + static_cast<int64_t>(layer0) * hkv * st->cap_blocks : nullptr,
      st->k_tscale ? st->k_tscale + layer0 * ts_ls : nullptr,
      st->v_tscale ? st->v_tscale + layer0 * ts_ls : nullptr,
      st->sink_k ? static_cast<uint16_t*>(st->sink_k) + layer0 * sink_ls : nullptr,
      st->sink_v ? static_cast<uint16_t*>(st->sink_v) + layer0 * sink_ls : nullptr, sink_ls,
      st->sink_tokens, sink_write_len);
  return launch_status("nkv_store_chunk");
}

extern "C" int nkv_build_reps(const nkv_store* st, int layer0, int num_layers, const uint16_t* k,
                              int64_t kv_layer_stride, int T, int start_block, void* stream) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_ARG(k != nullptr, "nkv_build_reps: k must be non-NULL");
  NKV_CHECK_ARG(T >= 1, "nkv_build_reps: T must be >= 1 (got %d)", T);
  const int nblk = (T + kBlock - 1) / kBlock;
  NKV_CHECK_ARG(start_block >= 0 && start_block + nblk <= st->cap_blocks,
                "nkv_build_reps: blocks [%d, %d) exceed cap_blocks %d", start_block, start_block + nblk,
                st->cap_blocks);
  const int64_t reps_ls = static_cast<int64_t>(st->num_kv_heads) * st->cap_blocks * st->r * kHeadDim;
  hipLaunchKernelGGL(build_reps_kernel, dim3(nblk, st->num_kv_heads, num_layers), dim3(kWave), 0,
                     reinterpret_cast<hipStream_t>(stream), k, kv_layer_stride, T, start_block,
                     st->num_kv_heads, st->cap_blocks, st->r,
                     static_cast<uint16_t*>(st->reps) + layer0 * reps_ls, reps_ls);
  return launch_status("nkv_build_reps");
}

extern "C" int nkv_recent_update(const nkv_store* st, int layer0, int num_layers, const uint16_t* k,
                                 const uint16_t* v, int64_t kv_layer_stride, int src_lo, int n_src,
                                 int ring_start, int old_len, int carry, void* stream) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  const int R = st->recent_tokens;
  NKV_CHECK_ARG(ring_start >= 0 && ring_start < R, "nkv_recent_update: ring_start %d outside [0, %d)", ring_start, R);
  NKV_CHECK_ARG(carry >= 0 && old_len >= carry && old_len <= R,
                "nkv_recent_update: need 0 <= carry <= old_len <= R (carry=%d, old_len=%d)", carry, old_len);
  NKV_CHECK_ARG(n_src >= 0 && src_lo >= 0 && carry + n_src <= R,
                "nkv_recent_update: carry + n_src must be <= R (carry=%d, n_src=%d)", carry, n_src);
  NKV_CHECK_ARG(n_src == 0 || (k != nullptr && v != nullptr), "nkv_recent_update: k/v are NULL");
  const int64_t rec_ls = static_cast<int64_t>(st->num_kv_heads) * R * kHeadDim;
  hipLaunchKernelGGL(recent_update_kernel, dim3(st->num_kv_heads, num_layers), dim3(kStoreThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), k, v, kv_layer_stride, src_lo, n_src, ring_start,
                     old_len, carry, st->num_kv_heads, R,
                     static_cast<uint16_t*>(st->recent_k) + layer0 * rec_ls,
                     static_cast<uint16_t*>(st->recent_v) + layer0 * rec_ls, rec_ls);
  return launch_status("nkv_recent_update");
}

extern "C" int nkv_query_summaries(const uint16_t* q, int64_t q_layer_stride, int num_layers, int T,
                                   int num_heads, int head_dim, int nsegments, uint16_t* out,
                                   int64_t out_layer_stride, void* stream) {
  NKV_CHECK_ARG(q != nullptr && out != nullptr, "nkv_query_summaries: q and out must be non-NULL");
  NKV_CHECK_ARG(T >= 1 && nsegments >= 1 && num_layers >= 1 && num_heads >= 1,
                "nkv_query_summaries: T, nsegments, num_layers and num_heads must be >= 1");
  NKV_CHECK_SUPPORTED(head_dim == kHeadDim, "nkv_query_summaries: head_dim must be %d", kHeadDim);
  const int nseg = nsegments < T ? nsegments : T;
  const int nelem = num_heads * head_dim;
  if ((reinterpret_cast<uintptr_t>(q) & 15u) == 0 && q_layer_stride % 8 == 0) {
    const int nc = nelem / 8;
    hipLaunchKernelGGL(query_mean8_kernel, dim3((nc + kQmChunks - 1) / kQmChunks, nseg, num_layers),
                       dim3(kStoreThreads), 0, reinterpret_cast<hipStream_t>(stream), q, q_layer_stride, T, nelem,
                       nseg, out, out_layer_stride);
  } else {
    hipLaunchKernelGGL(query_mean_kernel, dim3((nelem + kStoreThreads - 1) / kStoreThreads, nseg, num_layers),
                       dim3(kStoreThreads), 0, reinterpret_cast<hipStream_t>(stream), q, q_layer_stride, T,
                       nelem, nseg, out, out_layer_stride);
  }
  return launch_status("nkv_query_summaries");
}
