// Block scoring and Top-K selection (kernels 1 and 2 of the layer-step).
//
// Kernel 1 (score_kernel) computes, per history block b,
//   score[b] = max_{n, h, g, j} dot(q[n][h*G+g], reps[h][b][j])
// with each 128-term dot accumulated by ONE lane in ascending d order with
// fp32 fma.  A bf16 x bf16 product is exact in fp32, so the result is a
// fixed, reproducible function of the inputs (the oracle restates it
// bit-for-bit).  Same math as the reference's Triton scorer
// (nanovllm/sparse/fused_select.py:23-54) and its eager einsum chain
// (nanovllm/sparse/m12_runtime.py:999-1003).
//
// Mapping: a wavefront owns 64 representative rows = 64/r blocks of one KV
// head.  The wave first streams that 16 KiB tile with fully coalesced 16-byte
// loads (lane i reads bytes [1024*c + 16*i, +16)), transposes it through LDS
// with an XOR swizzle (conflict-free ds_read_b128), and then every lane dots
// its own row with the G query rows of that head; the query values are
// wave-uniform, so they are read with scalar loads.  Block maxima across the
// r rows use lane shuffles; across heads a running max per lane; across the
// two waves of a workgroup LDS.
//
// Kernel 2 (topk_kernel) selects, per (layer[, query]), the k largest scores
// with protected blocks forced to -inf: an LDS radix select over the 32-bit
// order-preserving key finds the k-th key T; one wavefront then collects
// keys > T and the lowest-id keys == T with ballots in ascending block order;
// a bitonic sort orders them (score desc, id asc).  Replaces
// m12_runtime.py:1004-1014 (protected mask) and :1033 (torch.topk).
#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kScoreWaves = 2;
constexpr int kScoreThreads = kScoreWaves * kWave;
constexpr int kTopkThreads = 256;
constexpr int kMaxTopk = 1024;
constexpr int kMaxSelectBlocks = 12288;  // keys + masks + sort buffer stay under 64 KiB of LDS
constexpr uint32_t kNegInfKey = 0x007fffffu;  // score_key(-inf)

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <int R, int G>
__global__ __launch_bounds__(kScoreThreads) void score_kernel(
    const uint16_t* __restrict__ q, int64_t q_ls, int nq, int per_query,
    const uint16_t* __restrict__ reps, int64_t reps_ls, int hkv, int cap,
    int nblocks, float* __restrict__ scores) {
  constexpr int TB = kWave / R;  // blocks per tile
  extern __shared__ uint4 smem[];
  uint4* stage = smem;  // [kScoreWaves][64 rows][16 chunks], swizzled
  float* red = reinterpret_cast<float*>(smem + kScoreWaves * 64 * 16);  // [waves][nq'][TB]

  const int nqo = per_query ? nq : 1;
  const int layer = blockIdx.y;
  const int b0 = blockIdx.x * TB;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int bl = lane / R;
  const int hq = hkv * G;
  const uint16_t* qL = q + static_cast<int64_t>(layer) * q_ls;
  const uint16_t* rL = reps + static_cast<int64_t>(layer) * reps_ls;

  for (int i = threadIdx.x; i < kScoreWaves * nqo * TB; i += kScoreThreads) red[i] = -INFINITY;
  __syncthreads();

  uint4* my = stage + wave * 64 * 16;
  float best = -INFINITY;
  const int n_iter = (hkv + kScoreWaves - 1) / kScoreWaves;
  for (int it = 0; it < n_iter; ++it) {
    const int h = wave + kScoreWaves * it;
    if (h >= hkv) break;  // wave-uniform
    const uint4* src = reinterpret_cast<const uint4*>(
        rL + (static_cast<int64_t>(h) * cap + b0) * R * kHeadDim);
    uint4 v[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int idx = c * 64 + lane;  // 16-byte chunk index inside the tile
      const int row = idx >> 4;
      v[c] = (b0 + row / R < nblocks) ? src[idx] : make_uint4(0u, 0u, 0u, 0u);
    }
    wave_lds_sync();  // previous head's reads of `my` are complete
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int idx = c * 64 + lane;
      const int row = idx >> 4, col = idx & 15;
      my[row * 16 + (col ^ (row & 15))] = v[c];
    }
    wave_lds_sync();

    for (int n = 0; n < nq; ++n) {
      const uint4* qh = reinterpret_cast<const uint4*>(
          qL + (static_cast<int64_t>(n) * hq + h * G) * kHeadDim);
      float acc[G];
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] = 0.0f;
#pragma unroll 2
      for (int c = 0; c < 16; ++c) {
        const uint4 rv = my[lane * 16 + (c ^ (lane & 15))];
        const float rf[8] = {bf16_lo(rv.x), bf16_hi(rv.x), bf16_lo(rv.y), bf16_hi(rv.y),
                             bf16_lo(rv.z), bf16_hi(rv.z), bf16_lo(rv.w), bf16_hi(rv.w)};
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint4 qv = qh[g * 16 + c];
          const float qf[8] = {bf16_lo(qv.x), bf16_hi(qv.x), bf16_lo(qv.y), bf16_hi(qv.y),
                               bf16_lo(qv.z), bf16_hi(qv.z), bf16_lo(qv.w), bf16_hi(qv.w)};
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g] = __builtin_fmaf(qf[e], rf[e], acc[g]);
        }
      }
      float m = acc[0];
#pragma unroll
      for (int g = 1; g < G; ++g) m = fmaxf(m, acc[g]);
#pragma unroll
      for (int o = 1; o < R; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
      if (per_query) {
        if ((lane % R) == 0) {
          float* slot = &red[(wave * nqo + n) * TB + bl];
          *slot = fmaxf(*slot, m);
        }
      } else {
        best = fmaxf(best, m);
      }
    }
  }
  if (!per_query && (lane % R) == 0) red[wave * TB + bl] = best;
  __syncthreads();
  for (int i = threadIdx.x; i < nqo * TB; i += kScoreThreads) {
    const int n = i / TB, b = i % TB;
    if (b0 + b < nblocks) {
      float m = red[n * TB + b];
#pragma unroll
      for (int w = 1; w < kScoreWaves; ++w) m = fmaxf(m, red[(w * nqo + n) * TB + b]);
      scores[(static_cast<int64_t>(layer) * nqo + n) * nblocks + b0 + b] = m;
    }
  }
}

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(
    const float* __restrict__ scores, int nblocks, const int32_t* __restrict__ prot,
    int nprot, int k_req, int order, int32_t* __restrict__ out_ids,
    float* __restrict__ out_vals, int k_stride) {
  extern __shared__ uint32_t sm[];
  uint32_t* keys = sm;                 // [nblocks]
  uint32_t* pmask = keys + nblocks;    // [ceil(nblocks / 32)]
  __shared__ uint32_t hist[256];
  __shared__ unsigned long long sel[kMaxTopk];
  __shared__ uint32_t s_digit, s_above, s_nprot;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const float* sc = scores + static_cast<int64_t>(row) * nblocks;
  const int nwords = (nblocks + 31) >> 5;

  if (tid == 0) {
    s_digit = 0u;
    s_above = 0u;
  }
  for (int i = tid; i < nwords; i += kTopkThreads) pmask[i] = 0u;
  for (int i = tid; i < nblocks; i += kTopkThreads) keys[i] = score_key(sc[i]);
  __syncthreads();
  for (int i = tid; i < nprot; i += kTopkThreads) {
    const int p = prot[i];
    if (p >= 0 && p < nblocks) {
      keys[p] = kNegInfKey;
      atomicOr(&pmask[p >> 5], 1u << (p & 31));
    }
  }
  __syncthreads();
  if (tid < 64) {
    uint32_t cnt = 0;
    for (int w = tid; w < nwords; w += 64) cnt += __popc(pmask[w]);
    for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o);
    if (tid == 0) s_nprot = cnt;
  }
  __syncthreads();
  const int avail = nblocks - static_cast<int>(s_nprot);
  const int k = min(k_req, max(1, avail));

  // ---- radix select of the k-th largest key, 8 bits per pass ------------
  uint32_t prefix = 0u, known = 0u;
  uint32_t remaining = static_cast<uint32_t>(k);
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0u;
    __syncthreads();
    for (int i = tid; i < nblocks; i += kTopkThreads) {
      const uint32_t key = keys[i];
      if ((key & known) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l owns digits 255-4l .. 252-4l (descending)
      uint32_t c[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) c[e] = hist[255 - 4 * lane - e];
      const uint32_t s = c[0] + c[1] + c[2] + c[3];
      uint32_t incl = s;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      const uint32_t excl = incl - s;
      if (excl < remaining && remaining <= incl) {
        uint32_t run = excl;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (run + c[e] >= remaining) {
            s_digit = static_cast<uint32_t>(255 - 4 * lane - e);
            s_above = run;
            break;
          }
          run += c[e];
        }
      }
    }
    __syncthreads();
    prefix |= s_digit << shift;
    known |= 0xffu << shift;
    remaining -= s_above;
    __syncthreads();
  }
  const uint32_t T = prefix;  // the k-th largest key; take `remaining` ties

  // ---- collect in ascending block order (one wavefront) ------------------
  if (tid < 64) {
    uint32_t base = 0u, need = remaining;
    const unsigned long long lt = (1ull << lane) - 1ull;
    for (int c0 = 0; c0 < nblocks; c0 += 64) {
      const int i = c0 + lane;
      const bool valid = i < nblocks;
      const uint32_t key = valid ? keys[i] : 0u;
      const bool gt = valid && key > T;
      const bool eq = valid && key == T;
      const unsigned long long meq = __ballot(eq);
      const uint32_t rank = __popcll(meq & lt);
      const bool take = gt || (eq && rank < need);
      const unsigned long long mt = __ballot(take);
      if (take) {
        const uint32_t pos = base + __popcll(mt & lt);
        sel[pos] = (static_cast<unsigned long long>(key) << 32) |
                   static_cast<unsigned long long>(0xffffffffu - static_cast<uint32_t>(i));
      }
      base += __popcll(mt);
      const uint32_t neq = __popcll(meq);
      need -= (neq < need ? neq : need);
    }
  }
  __syncthreads();

  if (order == NKV_ORDER_SCORE_DESC && k > 1) {
    int n2 = 1;
    while (n2 < k) n2 <<= 1;
    for (int i = k + tid; i < n2; i += kTopkThreads) sel[i] = 0ull;
    __syncthreads();
    for (int size = 2; size <= n2; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < (n2 >> 1); i += kTopkThreads) {
          const int lo = 2 * i - (i & (stride - 1));
          const int hi = lo + stride;
          const bool desc = (lo & size) == 0;
          const unsigned long long a = sel[lo], b = sel[hi];
          if (desc ? (a < b) : (a > b)) {
            sel[lo] = b;
            sel[hi] = a;
          }
        }
        __syncthreads();
      }
    }
  }
  for (int i = tid; i < k; i += kTopkThreads) {
    const unsigned long long e = sel[i];
    const int64_t o = static_cast<int64_t>(row) * k_stride + i;
    out_ids[o] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(e & 0xffffffffull));
    if (out_vals) out_vals[o] = key_score(static_cast<uint32_t>(e >> 32));
  }
}

template <int R, int G>
void launch_score(dim3 grid, size_t smem, hipStream_t s, const uint16_t* q, int64_t q_ls, int nq,
                  int per_query, const uint16_t* reps, int64_t reps_ls, int hkv, int cap,
                  int nblocks, float* scores) {
  hipLaunchKernelGGL((score_kernel<R, G>), grid, dim3(kScoreThreads), smem, s, q, q_ls, nq,
                     per_query, reps, reps_ls, hkv, cap, nblocks, scores);
}

template <int R>
int dispatch_g(int g, dim3 grid, size_t smem, hipStream_t s, const uint16_t* q, int64_t q_ls,
               int nq, int per_query, const uint16_t* reps, int64_t reps_ls, int hkv, int cap,
               int nblocks, float* scores) {
  switch (g) {
    case 1: launch_score<R, 1>(grid, smem, s, q, q_ls, nq, per_query, reps, reps_ls, hkv, cap, nblocks, scores); return 0;
    case 2: launch_score<R, 2>(grid, smem, s, q, q_ls, nq, per_query, reps, reps_ls, hkv, cap, nblocks, scores); return 0;
    case 4: launch_score<R, 4>(grid, smem, s, q, q_ls, nq, per_query, reps, reps_ls, hkv, cap, nblocks, scores); return 0;
    case 8: launch_score<R, 8>(grid, smem, s, q, q_ls, nq, per_query, reps, reps_ls, hkv, cap, nblocks, scores); return 0;
    case 16: launch_score<R, 16>(grid, smem, s, q, q_ls, nq, per_query, reps, reps_ls, hkv, cap, nblocks, scores); return 0;
    default: return -1;
  }
}

}  // namespace
}  // namespace nkv

using namespace nkv;

extern "C" int nkv_select(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                          int64_t q_layer_stride, int nq, int per_query, int nblocks,
                          const int32_t* protected_ids, int n_protected, int k, int order,
                          float* scores_ws, int32_t* out_ids, float* out_vals, void* stream) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_ARG(q != nullptr && scores_ws != nullptr && out_ids != nullptr,
                "nkv_select: q, scores_ws and out_ids must be non-NULL");
  NKV_CHECK_ARG(nq >= 1 && nq <= 64, "nkv_select: nq must be in [1, 64] (got %d)", nq);
  NKV_CHECK_ARG(!per_query || nq <= 16, "nkv_select: per-query selection supports nq <= 16 (got %d)", nq);
  NKV_CHECK_ARG(nblocks >= 1, "nkv_select: selection needs at least one history block (nblocks=%d)", nblocks);
  NKV_CHECK_ARG(nblocks <= st->cap_blocks, "nkv_select: nblocks %d exceeds cap_blocks %d", nblocks, st->cap_blocks);
  NKV_CHECK_SUPPORTED(nblocks <= kMaxSelectBlocks, "nkv_select: nblocks %d exceeds %d", nblocks, kMaxSelectBlocks);
  NKV_CHECK_ARG(k >= 1 && k <= kMaxTopk, "nkv_select: k must be in [1, %d] (got %d)", kMaxTopk, k);
  NKV_CHECK_ARG(n_protected >= 0 && (n_protected == 0 || protected_ids != nullptr),
                "nkv_select: protected list is NULL but n_protected=%d", n_protected);
  NKV_CHECK_ARG(order == NKV_ORDER_SCORE_DESC || order == NKV_ORDER_ID_ASC, "nkv_select: unknown order %d", order);
  NKV_CHECK_ARG(q_layer_stride >= static_cast<int64_t>(nq) * st->num_heads * kHeadDim || num_layers == 1,
                "nkv_select: q_layer_stride too small");

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int g = st->num_heads / st->num_kv_heads;
  const int R = st->r;
  const int TB = kWave / R;
  const int nqo = per_query ? nq : 1;
  const int64_t reps_ls = static_cast<int64_t>(st->num_kv_heads) * st->cap_blocks * R * kHeadDim;
  const uint16_t* reps = static_cast<const uint16_t*>(st->reps) + layer0 * reps_ls;
  dim3 grid((nblocks + TB - 1) / TB, num_layers);
  const size_t smem = kScoreWaves * 64 * 16 * sizeof(uint4) + kScoreWaves * nqo * TB * sizeof(float);
  int bad = 0;
  switch (R) {
    case 1: bad = dispatch_g<1>(g, grid, smem, s, q, q_layer_stride, nq, per_query, reps, reps_ls, st->num_kv_heads, st->cap_blocks, nblocks, scores_ws); break;
    case 2: bad = dispatch_g<2>(g, grid, smem, s, q, q_layer_stride, nq, per_query, reps, reps_ls, st->num_kv_heads, st->cap_blocks, nblocks, scores_ws); break;
    case 4: bad = dispatch_g<4>(g, grid, smem, s, q, q_layer_stride, nq, per_query, reps, reps_ls, st->num_kv_heads, st->cap_blocks, nblocks, scores_ws); break;
    case 8: bad = dispatch_g<8>(g, grid, smem, s, q, q_layer_stride, nq, per_query, reps, reps_ls, st->num_kv_heads, st->cap_blocks, nblocks, scores_ws); break;
    default: bad = -1;
  }
  NKV_CHECK_SUPPORTED(bad == 0, "nkv_select: unsupported (r=%d, G=%d)", R, g);
  rc = launch_status("nkv_select/score");
  if (rc != NKV_OK) return rc;

  const int nwords = (nblocks + 31) >> 5;
  const size_t tsmem = static_cast<size_t>(nblocks + nwords) * sizeof(uint32_t);
  hipLaunchKernelGGL(topk_kernel, dim3(num_layers * nqo), dim3(kTopkThreads), tsmem, s, scores_ws,
                     nblocks, protected_ids, n_protected, k, order, out_ids, out_vals, k);
  return launch_status("nkv_select/topk");
}
