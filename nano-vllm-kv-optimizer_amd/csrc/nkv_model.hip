// Fused elementwise kernels of the Qwen3 decoder around the sparse
// layer-step (its caller: nanovllm/models/qwen3.py).
//
// One launch each for what the reference runs as a chain of small tensor
// ops, with the same rounding points (fp32 arithmetic, bf16 where the
// reference stores a bf16 tensor):
//  * rmsnorm_kernel: RMSNorm, optionally after the residual add
//    (nanovllm/layers/layernorm.py:17-44): s = x (+ r) in fp32,
//    r' = bf16(s), y = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * w);
//  * qk_norm_rope_kernel: per-head RMSNorm of q and k, then rotate-half RoPE
//    in fp32 with the products and sums rounded separately, as separate
//    tensor ops round them (nanovllm/models/qwen3.py:99-110,
//    nanovllm/layers/rotary_embedding.py:6-50); v is copied out of the
//    fused projection output so that q, k and v are contiguous;
//  * silu_mul_kernel: SiLU(gate) * up (nanovllm/layers/activation.py:6-11),
//    bf16(bf16(g / (1 + e^-g)) * u).
//  * gemv_kernel: the decode-time projections (nn.Linear without bias on
//    1-4 rows, nanovllm/layers/linear.py) as an HBM-bound matrix-vector
//    product, fp32 accumulation, bf16 output.
// The sums of squares are taken in a fixed order of this kernel's own, so
// a result can differ from a tensor library's reduction by an fp32 rounding.
#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;  // 8-element chunks per thread: rows of up to 8192
constexpr int kMaxNormWidth = kNormThreads * kNormChunks * 8;

__device__ __forceinline__ void unpack8(const uint4& c, float (&f)[8]) {
  f[0] = bf16_lo(c.x); f[1] = bf16_hi(c.x);
  f[2] = bf16_lo(c.y); f[3] = bf16_hi(c.y);
  f[4] = bf16_lo(c.z); f[5] = bf16_hi(c.z);
  f[6] = bf16_lo(c.w); f[7] = bf16_hi(c.w);
}

__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  uint32_t u[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    u[i] = static_cast<uint32_t>(f32_to_bf16(f[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(f[2 * i + 1])) << 16);
  return make_uint4(u[0], u[1], u[2], u[3]);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// One workgroup per row.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, uint16_t* __restrict__ res_out, int n, float eps) {
  __shared__ float s_part[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  const int nc = n >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * n);
  const uint4* rr = res ? reinterpret_cast<const uint4*>(res + row * n) : nullptr;
  uint4* ro = res_out ? reinterpret_cast<uint4*>(res_out + row * n) : nullptr;
  float v[kNormChunks][8];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < nc) {
      unpack8(xr[c], v[j]);
      if (rr) {
        float r[8];
        unpack8(rr[c], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] += r[e];
      }
      if (ro) ro[c] = pack8(v[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
    }
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) s_part[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) tot += s_part[i];
  const float r = rsqrtf(tot / static_cast<float>(n) + eps);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* yr = reinterpret_cast<uint4*>(y + row * n);
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < nc) {
      float wf[8], o[8];
      unpack8(wr[c], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = round_bf16(v[j][e] * r) * wf[e];
      yr[c] = pack8(o);
    }
  }
}

// One wavefront per (token, head) of the fused q|k|v projection output; lane
// l holds dims l and l + 64, which is exactly one rotate-half RoPE pair.
constexpr int kRopeWaves = 4;
__global__ __launch_bounds__(kRopeWaves * kWave) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, int hq, int hkv, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    int max_pos, const int64_t* __restrict__ positions, float eps, uint16_t* __restrict__ q,
    uint16_t* __restrict__ k, uint16_t* __restrict__ v) {
#pragma clang fp contract(off)
  const int64_t t = blockIdx.x;
  const int nh = hq + 2 * hkv;
  const int head = blockIdx.y * kRopeWaves + static_cast<int>(threadIdx.x / kWave);
  if (head >= nh) return;
  const int lane = threadIdx.x & (kWave - 1);
  const uint16_t* src = qkv + (t * nh + head) * kHeadDim;
  if (head >= hq + hkv) {
    uint16_t* dst = v + (t * hkv + (head - hq - hkv)) * kHeadDim;
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
    return;
  }
  const bool isq = head < hq;
  const float a0 = bf16_to_f32(src[lane]);
  const float b0 = bf16_to_f32(src[lane + 64]);
  float ss = a0 * a0 + b0 * b0;
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float r = rsqrtf(ss * (1.0f / kHeadDim) + eps);
  const uint16_t* wv = isq ? qw : kw;
  const float a = round_bf16(round_bf16(a0 * r) * bf16_to_f32(wv[lane]));
  const float b = round_bf16(round_bf16(b0 * r) * bf16_to_f32(wv[lane + 64]));
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const float c = cos_t[pos * (kHeadDim / 2) + lane];
  const float s = sin_t[pos * (kHeadDim / 2) + lane];
  const float y1 = a * c - b * s;
  const float y2 = b * c + a * s;
  uint16_t* dst = isq ? q + (t * hq + head) * kHeadDim : k + (t * hkv + (head - hq)) * kHeadDim;
  dst[lane] = f32_to_bf16(y1);
  dst[lane + 64] = f32_to_bf16(y2);
}

// One thread per 8 outputs.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                       int64_t chunks, int inter) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= chunks) return;
  const int per_row = inter >> 3;
  const int64_t row = i / per_row;
  const int c = static_cast<int>(i % per_row);
  const uint16_t* g0 = gu + row * 2 * inter;
  float g[8], u[8], o[8];
  unpack8(reinterpret_cast<const uint4*>(g0)[c], g);
  unpack8(reinterpret_cast<const uint4*>(g0 + inter)[c], u);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = round_bf16(g[e] / (1.0f + expf(-g[e]))) * u[e];
  reinterpret_cast<uint4*>(out + row * inter)[c] = pack8(o);
}

// y[m][r] = sum_k x[m][k] w[r][k] (nn.Linear without bias) for up to 4 rows
// of x.  A workgroup owns ROWS weight rows; its 4 wavefronts take a quarter
// of k each, every lane streaming one 16-byte chunk of each row per
// iteration with the matching x chunk (L1 / L2 hits); fp32 fma
// accumulation, a wavefront sum, then the 4 quarters summed through LDS in
// wavefront order.  One chunk per row in flight keeps the wave small (more
// resident wavefronts per CU), which on gfx950 streams the weights faster
// than deeper per-wave unrolling: 5.5-5.8 TB/s on a 19456 x 2560 matrix
// against 2.7 TB/s with 8 chunks per row in flight.  HBM-bound: the weight
// matrix is read once.  The per-lane chunk order and the reduction order
// depend only on k, so a row's sum is the same for every ROWS.
constexpr int kGemvRows = 2;      // plain GEMV: rows per workgroup
constexpr int kGemvSiluRows = 4;  // gate|up: 2 gate rows + the 2 matching up rows

__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float acc) {
  float fa[8], fb[8];
  unpack8(a, fa);
  unpack8(b, fb);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(fa[e], fb[e], acc);
  return acc;
}

// SILU: w is the fused gate|up weight [2 n][k]; the workgroup's rows are gate
// rows r0 .. r0 + ROWS/2 - 1 and the matching up rows n + r0 ..; the epilogue
// writes bf16(bf16(silu(bf16 g)) * bf16 u) for rows r0 .. of y [m][n] (the
// rounding points of a bf16 GEMM followed by nkv_silu_mul).
template <int MR, int ROWS, bool SILU = false>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ w, const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ y, int n, int k) {
  constexpr int kOut = SILU ? ROWS / 2 : ROWS;  // output rows per workgroup
  __shared__ float s_red[4][MR][ROWS];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int r0 = blockIdx.x * kOut;
  const int nc = k >> 3;
  const int cbeg = static_cast<int>(static_cast<int64_t>(nc) * wave / 4);
  const int cend = static_cast<int>(static_cast<int64_t>(nc) * (wave + 1) / 4);
  const uint4* wr[ROWS];
#pragma unroll
  for (int j = 0; j < ROWS; ++j) {
    // rows past n re-read the last row (not stored)
    const int r = SILU ? min(r0 + j % kOut, n - 1) + (j / kOut) * n : min(r0 + j, n - 1);
    wr[j] = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(r) * k);
  }
  const uint4* xv = reinterpret_cast<const uint4*>(x);
  float acc[MR][ROWS];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < ROWS; ++j) acc[m][j] = 0.0f;
  for (int c = cbeg + lane; c < cend; c += kWave) {
    uint4 a[ROWS];
#pragma unroll
    for (int j = 0; j < ROWS; ++j) a[j] = wr[j][c];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const uint4 xm = xv[static_cast<int64_t>(m) * nc + c];
#pragma unroll
      for (int j = 0; j < ROWS; ++j) acc[m][j] = dot8(a[j], xm, acc[m][j]);
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int j = 0; j < ROWS; ++j)
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) acc[m][j] += __shfl_xor(acc[m][j], o);
  if (lane == 0)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int j = 0; j < ROWS; ++j) s_red[wave][m][j] = acc[m][j];
  __syncthreads();
  if (threadIdx.x >= MR * kOut) return;
  const int m = threadIdx.x / kOut, j = threadIdx.x % kOut;
  if (r0 + j >= n) return;
  const float v = s_red[0][m][j] + s_red[1][m][j] + s_red[2][m][j] + s_red[3][m][j];
  if constexpr (SILU) {
    const float g = round_bf16(v);
    const float u = round_bf16(s_red[0][m][kOut + j] + s_red[1][m][kOut + j] + s_red[2][m][kOut + j] +
                               s_red[3][m][kOut + j]);
    y[static_cast<int64_t>(m) * n + r0 + j] = f32_to_bf16(round_bf16(g / (1.0f + expf(-g))) * u);
  } else {
    y[static_cast<int64_t>(m) * n + r0 + j] = f32_to_bf16(v);
  }
}

template <int MR>
void launch_gemv_silu(const uint16_t* w, const uint16_t* x, uint16_t* y, int n, int k, hipStream_t s) {
  constexpr int rows_per_wg = kGemvSiluRows / 2;
  hipLaunchKernelGGL((gemv_kernel<MR, kGemvSiluRows, true>), dim3((n + rows_per_wg - 1) / rows_per_wg), dim3(256), 0,
                     s, w, x, y, n, k);
}

template <int MR>
void launch_gemv(const uint16_t* w, const uint16_t* x, uint16_t* y, int n, int k, hipStream_t s) {
  hipLaunchKernelGGL((gemv_kernel<MR, kGemvRows>), dim3((n + kGemvRows - 1) / kGemvRows), dim3(256), 0, s, w, x, y, n,
                     k);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace nkv

using namespace nkv;

extern "C" int nkv_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, uint16_t* out,
                           uint16_t* residual_out, int rows, int n, float eps, void* stream) {
  NKV_CHECK_ARG(x != nullptr && weight != nullptr && out != nullptr, "nkv_rmsnorm: x, weight and out must be non-NULL");
  NKV_CHECK_ARG(rows >= 1, "nkv_rmsnorm: rows must be >= 1 (got %d)", rows);
  NKV_CHECK_ARG(n >= 8 && n % 8 == 0 && n <= kMaxNormWidth, "nkv_rmsnorm: n must be a multiple of 8 in [8, %d] (got %d)",
                kMaxNormWidth, n);
  NKV_CHECK_ARG(aligned16(x) && aligned16(weight) && aligned16(out) && (!residual || aligned16(residual)) &&
                    (!residual_out || aligned16(residual_out)),
                "nkv_rmsnorm: every buffer must be 16-byte aligned");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, reinterpret_cast<hipStream_t>(stream), x,
                     residual, weight, out, residual_out, n, eps);
  return launch_status("nkv_rmsnorm");
}

extern "C" int nkv_qk_norm_rope(const uint16_t* qkv, int rows, int num_heads, int num_kv_heads, const uint16_t* q_weight,
                                const uint16_t* k_weight, const float* cos_table, const float* sin_table,
                                int max_position, const int64_t* positions, float eps, uint16_t* q, uint16_t* k,
                                uint16_t* v, void* stream) {
  NKV_CHECK_ARG(qkv != nullptr && q_weight != nullptr && k_weight != nullptr && cos_table != nullptr &&
                    sin_table != nullptr && positions != nullptr && q != nullptr && k != nullptr && v != nullptr,
                "nkv_qk_norm_rope: every pointer must be non-NULL");
  NKV_CHECK_ARG(rows >= 1 && num_heads >= 1 && num_kv_heads >= 1 && max_position >= 1,
                "nkv_qk_norm_rope: rows, heads and max_position must be >= 1");
  const int nh = num_heads + 2 * num_kv_heads;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(rows, (nh + kRopeWaves - 1) / kRopeWaves), dim3(kRopeWaves * kWave), 0,
                     reinterpret_cast<hipStream_t>(stream), qkv, num_heads, num_kv_heads, q_weight, k_weight,
                     cos_table, sin_table, max_position, positions, eps, q, k, v);
  return launch_status("nkv_qk_norm_rope");
}

extern "C" int nkv_silu_mul(const uint16_t* gate_up, uint16_t* out, int rows, int intermediate, void* stream) {
  NKV_CHECK_ARG(gate_up != nullptr && out != nullptr, "nkv_silu_mul: gate_up and out must be non-NULL");
  NKV_CHECK_ARG(rows >= 1 && intermediate >= 8 && intermediate % 8 == 0,
                "nkv_silu_mul: rows >= 1 and intermediate a positive multiple of 8 (got %d, %d)", rows, intermediate);
  NKV_CHECK_ARG(aligned16(gate_up) && aligned16(out), "nkv_silu_mul: buffers must be 16-byte aligned");
  const int64_t chunks = static_cast<int64_t>(rows) * (intermediate / 8);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), gate_up, out, chunks, intermediate);
  return launch_status("nkv_silu_mul");
}

extern "C" int nkv_gemv(const uint16_t* weight, const uint16_t* x, uint16_t* y, int m, int n, int k, void* stream) {
  NKV_CHECK_ARG(weight != nullptr && x != nullptr && y != nullptr, "nkv_gemv: weight, x and y must be non-NULL");
  NKV_CHECK_ARG(m >= 1 && m <= 4, "nkv_gemv: m must be in [1, 4] (got %d)", m);
  NKV_CHECK_ARG(n >= 1 && k >= 8 && k % 8 == 0, "nkv_gemv: n >= 1 and k a positive multiple of 8 (got %d, %d)", n, k);
  NKV_CHECK_ARG(aligned16(weight) && aligned16(x), "nkv_gemv: weight and x must be 16-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (m) {
    case 1: launch_gemv<1>(weight, x, y, n, k, s); break;
    case 2: launch_gemv<2>(weight, x, y, n, k, s); break;
    case 3: launch_gemv<3>(weight, x, y, n, k, s); break;
    default: launch_gemv<4>(weight, x, y, n, k, s); break;
  }
  return launch_status("nkv_gemv");
}

extern "C" int nkv_gemv_silu_mul(const uint16_t* gate_up_weight, const uint16_t* x, uint16_t* y, int m,
                                 int intermediate, int k, void* stream) {
  NKV_CHECK_ARG(gate_up_weight != nullptr && x != nullptr && y != nullptr,
                "nkv_gemv_silu_mul: gate_up_weight, x and y must be non-NULL");
  NKV_CHECK_ARG(m >= 1 && m <= 4, "nkv_gemv_silu_mul: m must be in [1, 4] (got %d)", m);
  NKV_CHECK_ARG(intermediate >= 1 && k >= 8 && k % 8 == 0,
                "nkv_gemv_silu_mul: intermediate >= 1 and k a positive multiple of 8 (got %d, %d)", intermediate, k);
  NKV_CHECK_ARG(aligned16(gate_up_weight) && aligned16(x), "nkv_gemv_silu_mul: weight and x must be 16-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (m) {
    case 1: launch_gemv_silu<1>(gate_up_weight, x, y, intermediate, k, s); break;
    case 2: launch_gemv_silu<2>(gate_up_weight, x, y, intermediate, k, s); break;
    case 3: launch_gemv_silu<3>(gate_up_weight, x, y, intermediate, k, s); break;
    default: launch_gemv_silu<4>(gate_up_weight, x, y, intermediate, k, s); break;
  }
  return launch_status("nkv_gemv_silu_mul");
}
