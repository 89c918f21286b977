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
// Mapping: a wavefront owns one (16-block tile, KV head) unit = 64 rows of
// r representatives; the 4 waves of a workgroup take 4 consecutive tiles of
// one KV head.  A wave streams its 16 KiB tile with 16-byte loads (each
// instruction reads 64-byte row quarters of 16 rows), transposes it through
// LDS a quarter at a time with an XOR swizzle (conflict-free ds_read_b128;
// 4 KiB of LDS per wave, so LDS does not bound the occupancy its 92 VGPRs
// allow), and then every lane dots
// its own row with the G query rows of that head, whose values come from
// scalar loads (wave-uniform) after one warm-up touch of their cache lines.
// Every vector load is unconditional (rows past nblocks are clamped and
// masked), so the waits count exactly.  Block maxima across the
// r rows use lane shuffles; the maximum across KV heads is an atomicMax on
// the order-preserving uint32 key of the score, which kernel 2 consumes and
// resets to zero.  Several queries (verify draft tokens, prefill tile
// summaries) take score_multi_kernel instead: one workgroup per two tiles,
// the query rows split over its four waves.
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

#ifndef NKV_SCORE_QLDS
#define NKV_SCORE_QLDS 1
#endif
constexpr bool kScoreQLds = NKV_SCORE_QLDS != 0;
constexpr int kScoreWaves = 4;
constexpr int kScoreThreads = kScoreWaves * kWave;
constexpr int kTopkThreads = 256;
constexpr int kMaxTopk = 1024;
constexpr int kMaxSelectBlocks = 12288;  // keys + masks + sort buffer stay under 64 KiB of LDS
constexpr uint32_t kNegInfKey = 0x007fffffu;  // score_key(-inf)
constexpr uint32_t kNaNKey = 0xffc00000u;     // score_key(NaN), above score_key(+inf)

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// x where keep holds, else zero, without turning the load of x into a
// conditional (exec-masked) one.
__device__ __forceinline__ uint4 and_mask(uint4 x, bool keep) {
  const uint32_t m = keep ? 0xffffffffu : 0u;
  return make_uint4(x.x & m, x.y & m, x.z & m, x.w & m);
}

// The G query rows of one (query, KV head): 16 G chunks of 8 bf16 at a
// wave-uniform address, read with scalar loads straight into the
// `v_fmac_f32 v, s, v` operand (no vector-ALU broadcast).  load() first touches
// every 64-byte line of the rows once, so the per-chunk scalar loads hit the
// scalar cache instead of queueing one line miss after another; the four
// waves of a workgroup score the same KV head, so they share those lines.
template <int G>
struct QueryChunks {
  const uint4* qh;   // the G rows of query n, KV head h: 16 G chunks of 16 bytes (uniform)

  __device__ __forceinline__ void load(const uint16_t* qL, int hq, int h, int n, int lane) {
    qh = reinterpret_cast<const uint4*>(qL + (static_cast<int64_t>(n) * hq + h * G) * kHeadDim);
    // bring every 64-byte line of the rows into the scalar cache at once
    uint32_t x = 0;
#pragma unroll
    for (int l = 0; l < 4 * G; ++l) x ^= reinterpret_cast<const uint32_t*>(qh)[l * 16];
    asm volatile("" ::"s"(x));
  }

  // acc[g] += q[g][8 c + e] * rv[e] for e = 0..7 in ascending order
  __device__ __forceinline__ void fma_chunk(const uint4& rv, int c, float (&acc)[G]) const {
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
};

// 64-bit sort/selection entry: key in the high word, ~id in the low word, so
// that a larger entry means a larger score, and on equal scores a lower id.
__device__ __forceinline__ unsigned long long sel_entry(uint32_t key, int id) {
  return (static_cast<unsigned long long>(key) << 32) |
         static_cast<unsigned long long>(0xffffffffu - static_cast<uint32_t>(id));
}

// Same selection as topk_kernel (identical ids, values and order) for one row
// of at most 64 J blocks, computed by ONE wavefront with no workgroup barrier
// (pmask: 2 J words of LDS, sel: LDS for max(k, 64) rounded up to a power of
// two entries).  Returns the number of ids written: k_req, or the number of
// selectable blocks when that is smaller (at least 1).
// Lane l holds the keys of blocks 64 j + l (j < J) in registers.  The k-th
// largest key T is found by a bitwise search of at most 32 steps: T is the
// largest value with count(key >= T) >= k, built from the high bit down, each
// count being J ballots.  Collection is the same ascending-id ballot pass as
// topk_kernel; up to 64 selected entries are then placed by their rank among
// the selection, larger k sorted by a bitonic network over LDS.
//
// STEP (the decode step's selection): the scorer left the protected blocks'
// keys at 0 (every scored key is >= score_key(-inf) > 0), and the step's
// attention launch zeroes the keys afterwards, so the row needs neither the
// protected list nor the zeroing stores; key 0 is read as score_key(-inf),
// exactly the protected mask of the general form.
template <int J, bool STEP>
__device__ __forceinline__ int select_row_wave(
    uint32_t* __restrict__ sk, int nblocks, const int32_t* __restrict__ prot, int nprot,
    int k_req, int order, int32_t* __restrict__ ids, float* __restrict__ vals,
    float* __restrict__ scores, uint32_t* pmask, unsigned long long* sel, int lane) {
  const int nwords = (nblocks + 31) >> 5;

  // The key reads go out first (they do not depend on the protected set), so
  // their latency overlaps the protected-id reads.  Keys past nblocks are 0,
  // below every key score_key() produces.  Every read is issued (past nblocks
  // it re-reads the last key), so one wait covers them all.
  uint32_t key[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = kWave * j + lane;
    key[j] = sk[i < nblocks ? i : nblocks - 1];
  }

  int avail = 0;
  if constexpr (STEP) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int i = kWave * j + lane;
      const bool valid = i < nblocks;
      avail += __popcll(__ballot(valid && key[j] != 0u));
      key[j] = !valid ? 0u : (key[j] == 0u ? kNegInfKey : key[j]);
    }
  } else {
    for (int w = lane; w < nwords; w += kWave) pmask[w] = 0u;
    wave_lds_sync();
    for (int i = lane; i < nprot; i += kWave) {
      const int p = prot[i];
      if (p >= 0 && p < nblocks) atomicOr(&pmask[p >> 5], 1u << (p & 31));
    }
    wave_lds_sync();

    // blocks in range and not protected, counted with ballots
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int i = kWave * j + lane;
      const bool valid = i < nblocks;
      const bool prot_i = valid && ((pmask[i >> 5] >> (i & 31)) & 1u);
      if (valid) {
        sk[i] = 0u;  // leave the key buffer zeroed for the next scoring pass
        if (scores) scores[i] = key_score(key[j]);
        if (prot_i) key[j] = kNegInfKey;
      } else {
        key[j] = 0u;
      }
      avail += __popcll(__ballot(valid && !prot_i));
    }
  }
  const int k = min(k_req, max(1, avail));

  // ---- fast path: rank a short candidate list -----------------------------
  // L0 = the k-th largest of the 64 lane maxima (one ballot per search step)
  // bounds the k-th largest key from below: k lanes hold a key >= L0.  Every
  // valid key >= L0 is a candidate; when there are at most 64 of them they
  // go to LDS in ascending block order and each lane ranks one against all
  // (the entries are distinct: the id is part of each), which places the
  // selection directly.  Otherwise (ties, adversarial spreads) the bitwise
  // search below runs over all keys.  Same selection either way.
  if (k <= kWave) {
    uint32_t lmax = key[0];
#pragma unroll
    for (int j = 1; j < J; ++j) lmax = max(lmax, key[j]);   // keys past nblocks are 0
    uint32_t L0 = 0u;
    for (uint32_t m = 0x80000000u; m != 0u; m >>= 1) {
      const uint32_t cand = L0 | m;
      const int cnt = __popcll(__ballot(lmax >= cand));
      if (cnt >= k) L0 = cand;
      if (cnt == k) break;
    }
    unsigned long long bc[J];
#pragma unroll
    for (int j = 0; j < J; ++j) bc[j] = __ballot(kWave * j + lane < nblocks && key[j] >= L0);
    int C = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) C += __popcll(bc[j]);
    if (C <= kWave) {
      const unsigned long long lt = (1ull << lane) - 1ull;
      int base = 0;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        if ((bc[j] >> lane) & 1ull) sel[base + __popcll(bc[j] & lt)] = sel_entry(key[j], kWave * j + lane);
        base += __popcll(bc[j]);
      }
      wave_lds_sync();
      // sel holds >= 64 entries, so the pair read at j = C - 1 stays inside it
      const unsigned long long e = sel[lane < C ? lane : 0];
      int rank = 0;
      const int cp = (C + 1) & ~1;
#pragma unroll 8
      for (int j = 0; j < cp; j += 2) {
        const unsigned long long a = sel[j], b = sel[j + 1];
        rank += (a > e) + ((j + 1 < C) & (b > e));
      }
      const bool chosen = lane < C && rank < k;
      int pos = rank;
      if (order != NKV_ORDER_SCORE_DESC) pos = __popcll(__ballot(chosen) & lt);   // ascending id
      if (chosen) {
        ids[pos] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(e & 0xffffffffull));
        if (vals) vals[pos] = key_score(static_cast<uint32_t>(e >> 32));
      }
      return k;
    }
  }

  // ---- k-th largest key: largest T with count(key >= T) >= k ------------
  // Once count(key >= T) == k the k keys >= T are the selection itself (every
  // key equal to the k-th largest is among them), so the search stops there:
  // the collection below then takes exactly those keys, as it would with the
  // fully resolved T.
  // T and the candidate stay scalar (one vector-to-scalar hand-off per
  // ballot, none back), and the J ballot counts are summed as a tree.
  uint32_t T = 0u;
  for (uint32_t m = 0x80000000u; m != 0u; m >>= 1) {
    const uint32_t cand = T | m;
    // all J compares issue before the first count reads one, so only the
    // first count waits for a compare result
    unsigned long long b[J];
#pragma unroll
    for (int j = 0; j < J; ++j) b[j] = __ballot(key[j] >= cand);
    __builtin_amdgcn_sched_barrier(0);
    int c[J];
#pragma unroll
    for (int j = 0; j < J; ++j) c[j] = __popcll(b[j]);
#pragma unroll
    for (int w = 1; w < J; w <<= 1)
#pragma unroll
      for (int j = 0; j + w < J; j += 2 * w) c[j] += c[j + w];
    const int cnt = c[0];
    if (cnt >= k) T = cand;
    if (cnt == k) break;
  }
  int above = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) above += __popcll(__ballot(key[j] > T));

  // ---- collect in ascending block order ----------------------------------
  const unsigned long long lt = (1ull << lane) - 1ull;
  uint32_t base = 0u;
  uint32_t need = static_cast<uint32_t>(k - above);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = kWave * j + lane;
    const bool gt = key[j] > T;
    const bool eq = key[j] == T && i < nblocks;
    const unsigned long long meq = __ballot(eq);
    const uint32_t rank = __popcll(meq & lt);
    const bool take = gt || (eq && rank < need);
    const unsigned long long mt = __ballot(take);
    if (take) sel[base + __popcll(mt & lt)] = sel_entry(key[j], i);
    base += __popcll(mt);
    const uint32_t neq = __popcll(meq);
    need -= (neq < need ? neq : need);
  }
  wave_lds_sync();

  if (order == NKV_ORDER_SCORE_DESC && k > 1 && k <= kWave) {
    // Rank sort: the entries are distinct (the id is part of each), so the
    // position of entry e in the descending order is the number of entries
    // larger than e.  Lane l < k ranks sel[l] against all k entries, read as
    // LDS broadcasts two at a time (sel holds at least 64 entries, so the
    // pair read at j = k - 1 stays inside it; its second entry is ignored).
    const unsigned long long e = sel[lane < k ? lane : 0];
    int rank = 0;
    const int kp = (k + 1) & ~1;
#pragma unroll 8
    for (int j = 0; j < kp; j += 2) {
      const unsigned long long a = sel[j], b = sel[j + 1];
      rank += (a > e) + ((j + 1 < k) & (b > e));
    }
    if (lane < k) {
      ids[rank] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(e & 0xffffffffull));
      if (vals) vals[rank] = key_score(static_cast<uint32_t>(e >> 32));
    }
    return k;
  }
  if (order == NKV_ORDER_SCORE_DESC && k > 1) {
    int n2 = 1;
    while (n2 < k) n2 <<= 1;
    for (int i = k + lane; i < n2; i += kWave) sel[i] = 0ull;
    wave_lds_sync();
    for (int size = 2; size <= n2; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = lane; i < (n2 >> 1); i += kWave) {
          const int lo = 2 * i - (i & (stride - 1));
          const int hi = lo + stride;
          const bool desc = (lo & size) == 0;
          const unsigned long long a = sel[lo], b = sel[hi];
          if (desc ? (a < b) : (a > b)) {
            sel[lo] = b;
            sel[hi] = a;
          }
        }
        wave_lds_sync();
      }
    }
  }
  for (int i = lane; i < k; i += kWave) {
    const unsigned long long e = sel[i];
    ids[i] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(e & 0xffffffffull));
    if (vals) vals[i] = key_score(static_cast<uint32_t>(e >> 32));
  }
  return k;
}


// The loaded operands of one (tile, head) unit: the 64 x 256 B tile of
// representative rows (16 x 16 B per lane) and the query chunks of query 0.
template <int G>
struct ScoreTile {
  uint4 v[16];
  QueryChunks<G> qc;
};

// Issues every load of unit `unit` of `layer` (no wait).  The tile is 64 rows
// x 256 B, read with 16-byte loads: load c holds dims 32 (c / 4) .. +31 (one
// 64-byte quarter) of rows 16 (c % 4) .. +15, lane l the chunk l % 4 of row
// 16 (c % 4) + l / 4.  Rows past nblocks are clamped to the last valid row
// and zeroed, so every load is issued.
template <int R, int G>
__device__ __forceinline__ void score_load(
    const uint16_t* __restrict__ q, int64_t q_ls, const uint16_t* __restrict__ reps,
    int64_t reps_ls, int hkv, int cap, int nblocks, int layer, int unit, int lane, ScoreTile<G>& t) {
  constexpr int TB = kWave / R;  // blocks per tile
  const int h = unit % hkv;
  const int b0 = (unit / hkv) * TB;
  const uint16_t* qL = q + static_cast<int64_t>(layer) * q_ls;
  const uint16_t* rL = reps + static_cast<int64_t>(layer) * reps_ls;
  const uint4* src = reinterpret_cast<const uint4*>(rL + (static_cast<int64_t>(h) * cap + b0) * R * kHeadDim);
  const int last_row = (nblocks - b0) * R - 1;  // rows past it belong to blocks >= nblocks
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    // quarter qt = c / 4 holds row chunks 4 qt .. 4 qt + 3; chunk index within
    // the tile: row * 16 + 4 qt + (i & 3) with i = (c % 4) * 64 + lane
    const int i = (c & 3) * 64 + lane;
    const int row = i >> 2;
    const int col = (c >> 2) * 4 + (i & 3);
    t.v[c] = and_mask(src[min(row, last_row) * 16 + col], row <= last_row);
  }
  t.qc.load(qL, hkv * G, h, 0, lane);
}

// The dots and block maxima of one loaded unit.  Per query n: dot over the
// four quarters in ascending d; each quarter is re-staged from registers
// through `my` (4 KiB of LDS per wave; against halves through 8 KiB: 36-layer
// 32K decode step +0.6-1.0%).
template <int R, int G>
__device__ __forceinline__ void score_dots(
    const uint16_t* __restrict__ q, int64_t q_ls, int nq, int per_query, int hkv, int nblocks,
    uint32_t* __restrict__ keys, int layer, int unit, int lane, ScoreTile<G>& t, uint4* my,
    const int32_t* __restrict__ skip_ids, int n_skip) {
  constexpr int TB = kWave / R;
  const int nqo = per_query ? nq : 1;
  const int h = unit % hkv;
  const int b = (unit / hkv) * TB + lane / R;
  const uint16_t* qL = q + static_cast<int64_t>(layer) * q_ls;
  uint32_t best = 0u;  // below every key score_key() produces
  for (int n = 0; n < nq; ++n) {
    if (n > 0) t.qc.load(qL, hkv * G, h, n, lane);
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      wave_lds_sync();  // previous quarter fully consumed
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = c * 64 + lane;
        const int row = i >> 2, col = i & 3;
        my[row * 4 + (col ^ ((row >> 2) & 3))] = t.v[qt * 4 + c];
      }
      wave_lds_sync();
      // two chunks per iteration for G <= 4 (the next chunk's reads issue
      // before the current products: decode step +0.3-0.9%); with more query
      // rows the second chunk's scalar operands would spill
      if constexpr (G <= 4) {
#pragma unroll 2
        for (int c = 0; c < 4; ++c) {
          const uint4 rv = my[lane * 4 + (c ^ ((lane >> 2) & 3))];
          t.qc.fma_chunk(rv, qt * 4 + c, acc);
        }
      } else {
#pragma unroll 1
        for (int c = 0; c < 4; ++c) {
          const uint4 rv = my[lane * 4 + (c ^ ((lane >> 2) & 3))];
          t.qc.fma_chunk(rv, qt * 4 + c, acc);
        }
      }
    }
    // the lane's maximum over its G dots, NaN if any of them is NaN (the
    // oracle's numpy max), then the key maximum over the block's r rows
    float m = acc[0];
    bool nan = __builtin_isnan(acc[0]);
#pragma unroll
    for (int g = 1; g < G; ++g) {
      m = fmaxf(m, acc[g]);
      nan |= __builtin_isnan(acc[g]);
    }
    uint32_t km = nan ? kNaNKey : score_key(m);
#pragma unroll
    for (int o = 1; o < R; o <<= 1) km = max(km, static_cast<uint32_t>(__shfl_xor(static_cast<int>(km), o)));
    if (per_query) {
      if ((lane % R) == 0 && b < nblocks)
        atomicMax(&keys[(static_cast<int64_t>(layer) * nqo + n) * nblocks + b], km);
    } else {
      best = max(best, km);
    }
  }
  if (!per_query) {
    // blocks on the skip list (the protected set, in the decode step) keep
    // key 0, which the step's top-k reads as "protected"
    bool skip = false;
    for (int i = 0; i < n_skip; ++i) skip |= skip_ids[i] == b;
    if ((lane % R) == 0 && b < nblocks && !skip)
      atomicMax(&keys[static_cast<int64_t>(layer) * nblocks + b], best);
  }
}

// One (tile, head) unit per wavefront (any nq).
template <int R, int G>
__global__ __launch_bounds__(kScoreThreads) void score_kernel(
    const uint16_t* __restrict__ q, int64_t q_ls, int nq, int per_query,
    const uint16_t* __restrict__ reps, int64_t reps_ls, int hkv, int cap,
    int nblocks, int units, uint32_t* __restrict__ keys, const int32_t* __restrict__ skip_ids, int n_skip) {
  __shared__ uint4 stage[kScoreWaves][64 * 4];  // per wave: 64 rows x 4 chunks (one quarter), swizzled
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // the 4 waves of a workgroup take 4 consecutive tiles of one KV head
  const int hh = blockIdx.x % hkv;
  const int tile = (blockIdx.x / hkv) * kScoreWaves + wave;
  const int unit = tile * hkv + hh;  // (tile, head) pair
  if (unit >= units) return;
  const int lane = threadIdx.x & 63;
  ScoreTile<G> t;
  score_load<R, G>(q, q_ls, reps, reps_ls, hkv, cap, nblocks, blockIdx.y, unit, lane, t);
  score_dots<R, G>(q, q_ls, nq, per_query, hkv, nblocks, keys, blockIdx.y, unit, lane, t, stage[wave], skip_ids,
                   n_skip);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(4))) const u32x4 cu32x4;  // read with scalar loads
typedef __attribute__((address_space(4))) const int32_t cint32;

// Multi-query form (nq >= 2: the draft tokens of a verify round, the tile
// summaries of a prefill chunk).  One workgroup per (32-block pair of tiles,
// KV head, layer): the 128 x 256 B of representative rows are copied into LDS
// with coalesced 16-byte loads (eight per thread) and the nq * G query rows
// of the head are split over the four waves, ceil(nq G / 4) rows each.  Every
// wave reads all the rows from LDS -- lane l owns rows l and 64 + l, widened
// to fp32 in registers -- and computes its share of the dots, QB query rows
// at a time: the same ascending-d fma chain from +0 as score_kernel
// (identical bits), each query value feeding both rows' products.  The
// query values (QLDS, the default) are widened to fp32 once per pass into
// the wave's own LDS area and read back as broadcasts (six-query 16K verify,
// 36 layers: 45.8 -> 40.0 us; 64-tile prefill selection +1.9% on the step);
// the other form scalar-loads them as bf16 and widens each with one scalar
// instruction, after touching the cache lines of the first query rows while
// the row loads are in flight.  Each wave's products are a quarter of the
// workgroup's and every SIMD gets the same number of waves.  Maxima are taken
// over the order-preserving keys: a query whose rows are split between two
// waves combines exactly through the atomicMax, and a NaN dot makes the
// block's score NaN (numpy's max).
template <int QB, bool QLDS>
__global__ __launch_bounds__(kScoreThreads) void score_multi_kernel(
    const uint16_t* __restrict__ q, int64_t q_ls, int nq, int per_query, int log_g,
    const uint16_t* __restrict__ reps, int64_t reps_ls, int hkv, int cap, int nblocks, int log_r,
    uint32_t* __restrict__ keys) {
  // row r (0 .. 127), dims 8c .. 8c+7 at r * 17 + c: the one-chunk pad per row
  // makes a lane-per-row ds_read_b128 conflict-free with an immediate offset
  __shared__ uint4 tile[2 * kWave * 17];
  // QLDS: each pass's QB query rows, widened to fp32, in the wave's own LDS
  // area (row i, dims 4 m .. 4 m + 3 at float4 i * 32 + m), read back as
  // broadcasts; otherwise the query values are scalar-loaded bf16 and
  // widened by scalar instructions, one per product pair
  __shared__ float4 qlds[QLDS ? kScoreWaves : 1][QLDS ? QB * 32 : 1];
  const int layer = blockIdx.y;
  const int h = blockIdx.x % hkv;
  const int R = 1 << log_r;
  const int TB = kWave >> log_r;  // blocks per 64 rows
  const int b0 = (blockIdx.x / hkv) * 2 * TB;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = 1 << log_g;
  const int J = nq << log_g;  // query rows (n, g), j = n G + g
  const int per = (J + kScoreWaves - 1) / kScoreWaves;
  const int j0 = wave * per;
  const int j1 = min(J, j0 + per);
  const int hq = hkv << log_g;
  const uint16_t* qL = q + static_cast<int64_t>(layer) * q_ls;
  auto qrow = [&](int j) {
    return reinterpret_cast<const char*>(
        qL + (static_cast<int64_t>(j >> log_g) * hq + (h << log_g) + (j & (G - 1))) * kHeadDim);
  };

  {
    // one dword of every 64-byte line of the wave's first QB query rows, read
    // first so that the scalar misses overlap the tile loads
    int32_t t[QB * 4];
#pragma unroll
    for (int i = 0; i < QB; ++i) {
      const cint32* r = (const cint32*)qrow(min(j0 + i, max(j1, 1) - 1));
#pragma unroll
      for (int l = 0; l < 4; ++l) t[4 * i + l] = QLDS ? 0 : r[16 * l];
    }
    // chunk i = k * 256 + tid of the 128 rows: row i / 16, dims 8 (i % 16)
    // .. +7; rows past nblocks are clamped to the last valid row and zeroed
    const uint4* src = reinterpret_cast<const uint4*>(
        reps + static_cast<int64_t>(layer) * reps_ls + (static_cast<int64_t>(h) * cap + b0) * (R * kHeadDim));
    const int last_row = ((nblocks - b0) << log_r) - 1;
    uint4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = k * kScoreThreads + tid;
      const int row = i >> 4;
      v[k] = and_mask(src[min(row, last_row) * 16 + (i & 15)], row <= last_row);
    }
    int32_t x = 0;
#pragma unroll
    for (int i = 0; i < QB * 4; ++i) x ^= t[i];
    asm volatile("" ::"s"(x));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = k * kScoreThreads + tid;
      tile[(i >> 4) * 17 + (i & 15)] = v[k];
    }
  }
  __syncthreads();

  // lane l owns rows l (block b0 + l / r) and 64 + l (TB blocks further)
  const int b = b0 + (lane >> log_r);
  const bool own0 = (lane & (R - 1)) == 0 && b < nblocks;
  const bool own1 = (lane & (R - 1)) == 0 && b + TB < nblocks;
  const uint4* my0 = tile + lane * 17;
  const uint4* my1 = tile + (lane + kWave) * 17;
  const int64_t krow = static_cast<int64_t>(layer) * (per_query ? nq : 1);

  // key maxima of the current query's rows in this lane (both rows), flushed
  // (maximum over the r rows of each block, then atomicMax) when the query
  // changes
  uint32_t cur0 = 0u, cur1 = 0u;
  int cur_n = -1;
  auto flush = [&](int n, uint32_t k0, uint32_t k1) {
    for (int o = 1; o < R; o <<= 1) {
      k0 = max(k0, static_cast<uint32_t>(__shfl_xor(static_cast<int>(k0), o)));
      k1 = max(k1, static_cast<uint32_t>(__shfl_xor(static_cast<int>(k1), o)));
    }
    if (own0) atomicMax(&keys[(krow + n) * nblocks + b], k0);
    if (own1) atomicMax(&keys[(krow + n) * nblocks + b + TB], k1);
  };
  for (int jg = j0; jg < j1; jg += QB) {
    const char* qp[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) qp[i] = qrow(min(jg + i, j1 - 1));  // a short last group repeats its last row
    if constexpr (QLDS) {
      // the previous pass's reads of the area are done before it is refilled
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      for (int idx = lane; idx < QB * 16; idx += kWave) {
        const int row = idx >> 4, ch = idx & 15;
        const uint4 w = *reinterpret_cast<const uint4*>(qrow(min(jg + row, j1 - 1)) + ch * 16);
        float4* dst = &qlds[wave][row * 32 + ch * 2];
        dst[0] = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
        dst[1] = make_float4(bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w));
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
    float acc0[QB], acc1[QB];
#pragma unroll
    for (int i = 0; i < QB; ++i) acc0[i] = acc1[i] = 0.0f;
    // 8 dims per pass: one 16-byte scalar load per query row at the shared
    // byte offset `off` (kept opaque so that each load addresses row + off
    // instead of stepping QB pointers), one chunk of each of the lane's rows
    // from LDS; every unpacked query value feeds two products
    uint32_t off = 0;
#pragma unroll 1
    for (int c = 0; c < 16; ++c) {
      asm volatile("" : "+s"(off));
      const uint4 va = my0[c], vb = my1[c];
      const float ra[8] = {bf16_lo(va.x), bf16_hi(va.x), bf16_lo(va.y), bf16_hi(va.y),
                           bf16_lo(va.z), bf16_hi(va.z), bf16_lo(va.w), bf16_hi(va.w)};
      const float rb[8] = {bf16_lo(vb.x), bf16_hi(vb.x), bf16_lo(vb.y), bf16_hi(vb.y),
                           bf16_lo(vb.z), bf16_hi(vb.z), bf16_lo(vb.w), bf16_hi(vb.w)};
#pragma unroll
      for (int i = 0; i < QB; ++i) {
        float qf[8];
        if constexpr (QLDS) {
          const float4 a = qlds[wave][i * 32 + 2 * c], b = qlds[wave][i * 32 + 2 * c + 1];
          qf[0] = a.x; qf[1] = a.y; qf[2] = a.z; qf[3] = a.w;
          qf[4] = b.x; qf[5] = b.y; qf[6] = b.z; qf[7] = b.w;
        } else {
          const u32x4 w = *(cu32x4*)(qp[i] + off);  // dims 8 c .. +7 of row jg + i
          qf[0] = bf16_lo(w.x); qf[1] = bf16_hi(w.x); qf[2] = bf16_lo(w.y); qf[3] = bf16_hi(w.y);
          qf[4] = bf16_lo(w.z); qf[5] = bf16_hi(w.z); qf[6] = bf16_lo(w.w); qf[7] = bf16_hi(w.w);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc0[i] = __builtin_fmaf(qf[e], ra[e], acc0[i]);
          acc1[i] = __builtin_fmaf(qf[e], rb[e], acc1[i]);
        }
      }
      off += 16;
    }
#pragma unroll
    for (int i = 0; i < QB; ++i) {
      const int j = jg + i;
      if (j >= j1) break;
      const int n = per_query ? (j >> log_g) : 0;
      const uint32_t k0 = score_key(acc0[i]), k1 = score_key(acc1[i]);
      if (n != cur_n) {
        if (cur_n >= 0) flush(cur_n, cur0, cur1);
        cur_n = n;
        cur0 = k0;
        cur1 = k1;
      } else {
        cur0 = max(cur0, k0);
        cur1 = max(cur1, k1);
      }
    }
  }
  if (cur_n >= 0) flush(cur_n, cur0, cur1);
}

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(
    uint32_t* __restrict__ score_keys, int nblocks, const int32_t* __restrict__ prot,
    int nprot, int k_req, int order, int32_t* __restrict__ out_ids,
    float* __restrict__ out_vals, int k_stride, float* __restrict__ out_scores) {
  extern __shared__ uint32_t sm[];
  uint32_t* keys = sm;                 // [nblocks]
  uint32_t* pmask = keys + nblocks;    // [ceil(nblocks / 32)]
  __shared__ uint32_t hist[256];
  __shared__ unsigned long long sel[kMaxTopk];
  __shared__ uint32_t s_digit, s_above, s_nprot;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  uint32_t* sk = score_keys + static_cast<int64_t>(row) * nblocks;
  const int nwords = (nblocks + 31) >> 5;

  if (tid == 0) {
    s_digit = 0u;
    s_above = 0u;
  }
  for (int i = tid; i < nwords; i += kTopkThreads) pmask[i] = 0u;
  for (int i = tid; i < nblocks; i += kTopkThreads) {
    const uint32_t key = sk[i];
    keys[i] = key;
    sk[i] = 0u;  // leave the key buffer zeroed for the next scoring pass
    if (out_scores) out_scores[static_cast<int64_t>(row) * nblocks + i] = key_score(key);
  }
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

// One wavefront per (layer[, query]) row.
template <int J, bool STEP>
__global__ __launch_bounds__(kWave) void topk_wave_kernel(
    uint32_t* __restrict__ score_keys, int nblocks, const int32_t* __restrict__ prot,
    int nprot, int k_req, int order, int32_t* __restrict__ out_ids,
    float* __restrict__ out_vals, int k_stride, float* __restrict__ out_scores) {
  __shared__ uint32_t pmask[J * 2];  // protected bitmap, one bit per block
  __shared__ unsigned long long sel[kMaxTopk];
  const int64_t row = blockIdx.x;
  select_row_wave<J, STEP>(score_keys + row * nblocks, nblocks, prot, nprot, k_req, order,
                     out_ids + row * k_stride, out_vals ? out_vals + row * k_stride : nullptr,
                     out_scores ? out_scores + row * nblocks : nullptr, pmask, sel, threadIdx.x);
}

constexpr int kUnionThreads = 256;
constexpr int kUnionMax = 4096;  // tq * k_eff ids per layer

// Union of one layer's per-query selections (one workgroup of NT threads per
// layer), through a bitmap of block ids in LDS: every selected id sets its
// bit, a prefix count over the bitmap words gives each set bit its position
// in the ascending union, and each query's ids find their mask columns by the
// same count.  Five barriers, no sort.  Ids are block ids of nkv_select
// (below kMaxSelectBlocks); any other value is left out of the union and the
// mask.  src: the layer's ids, row t at src + t * k (global memory, or LDS
// for the fused top-k + union).
constexpr int kUnionWords = kMaxSelectBlocks / 32;
template <int NT>
struct UnionLds {
  uint32_t bits[kUnionWords];
  int32_t pre[kUnionWords];   // set bits in the words before
  int32_t wsum[NT / kWave];
  int32_t s_max;
};

template <int NT>
__device__ __forceinline__ void union_layer(const int32_t* src, int layer, int tq, int k, int k_eff, int umax,
                                            int32_t* __restrict__ out_union, int32_t* __restrict__ out_count,
                                            uint8_t* __restrict__ out_allowed, UnionLds<NT>& sh, int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  const int n = tq * k_eff;
  auto id_at = [&](int i) { return src[(i / k_eff) * k + i % k_eff]; };
  auto valid = [](int32_t id) { return id >= 0 && id < kMaxSelectBlocks; };

  // the largest id bounds the words to clear and count
  int32_t mx = -1;
  for (int i = tid; i < n; i += NT) {
    const int32_t id = id_at(i);
    if (valid(id)) mx = max(mx, id);
  }
  for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o));
  if (tid == 0) sh.s_max = -1;
  __syncthreads();
  if (lane == 0) atomicMax(&sh.s_max, mx);
  __syncthreads();
  const int nwords = (sh.s_max + 32) >> 5;   // 0 when no id is valid
  for (int w = tid; w < nwords; w += NT) sh.bits[w] = 0u;
  __syncthreads();
  for (int i = tid; i < n; i += NT) {
    const int32_t id = id_at(i);
    if (valid(id)) atomicOr(&sh.bits[id >> 5], 1u << (id & 31));
  }
  __syncthreads();

  // exclusive prefix count of set bits over the words (thread t owns a
  // contiguous run of words)
  const int per = (nwords + NT - 1) / NT;
  const int w0 = min(tid * per, nwords), w1 = min(w0 + per, nwords);
  int cnt = 0;
  for (int w = w0; w < w1; ++w) cnt += __popc(sh.bits[w]);
  int incl = cnt;
  for (int o = 1; o < kWave; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  if (lane == kWave - 1) sh.wsum[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += sh.wsum[w];
  int run = base + incl - cnt;
  for (int w = w0; w < w1; ++w) {
    sh.pre[w] = run;
    run += __popc(sh.bits[w]);
  }
  int U = 0;
  for (int w = 0; w < NT / kWave; ++w) U += sh.wsum[w];
  __syncthreads();

  // the union, ascending, then -1
  int32_t* ou = out_union + static_cast<int64_t>(layer) * umax;
  for (int w = tid; w < nwords; w += NT) {
    uint32_t b = sh.bits[w];
    int pos = sh.pre[w];
    while (b != 0u) {
      const int bit = __builtin_ctz(b);
      ou[pos++] = 32 * w + bit;
      b &= b - 1u;
    }
  }
  for (int i = U + tid; i < umax; i += NT) ou[i] = -1;
  if (tid == 0) out_count[layer] = U;

  // mask rows: zeros, then each query's ids at their union positions
  uint8_t* oa = out_allowed + static_cast<int64_t>(layer) * tq * umax;
  for (int i = tid; i < tq * umax; i += NT) oa[i] = 0;
  __syncthreads();  // the zeros are written before the ones
  for (int i = tid; i < n; i += NT) {
    const int32_t id = id_at(i);
    if (!valid(id)) continue;
    const int pos = sh.pre[id >> 5] + __popc(sh.bits[id >> 5] & ((1u << (id & 31)) - 1u));
    oa[static_cast<int64_t>(i / k_eff) * umax + pos] = 1;
  }
}

__global__ __launch_bounds__(kUnionThreads) void union_kernel(
    const int32_t* __restrict__ ids, int tq, int k, int k_eff, int umax, int32_t* __restrict__ out_union,
    int32_t* __restrict__ out_count, uint8_t* __restrict__ out_allowed) {
  __shared__ UnionLds<kUnionThreads> sh;
  const int layer = blockIdx.x;
  union_layer<kUnionThreads>(ids + static_cast<int64_t>(layer) * tq * k, layer, tq, k, k_eff, umax, out_union,
                             out_count, out_allowed, sh, threadIdx.x);
}

// Per-query Top-K and their union in one launch (one workgroup per layer):
// wavefront w selects rows w, w + kFusedWaves, ... of the layer (the same
// selection as topk_wave_kernel, written to out_ids / out_vals / out_scores
// and kept in LDS), then the workgroup forms the union and mask of those ids
// as union_kernel does.  For k <= 64 and at most 16 queries.
constexpr int kFusedWaves = 8;
constexpr int kFusedMaxK = kWave;
constexpr int kFusedMaxQ = 16;
template <int J>
__global__ __launch_bounds__(kFusedWaves * kWave) void topk_union_kernel(
    uint32_t* __restrict__ score_keys, int nblocks, const int32_t* __restrict__ prot, int nprot, int k_req, int tq,
    int order, int32_t* __restrict__ out_ids, float* __restrict__ out_vals, float* __restrict__ out_scores, int umax,
    int32_t* __restrict__ out_union, int32_t* __restrict__ out_count, uint8_t* __restrict__ out_allowed) {
  __shared__ uint32_t pmask[kFusedWaves][J * 2];
  __shared__ unsigned long long sel[kFusedWaves][kFusedMaxK];
  __shared__ int32_t sids[kFusedMaxQ * kFusedMaxK];
  __shared__ int32_t s_keff;
  __shared__ UnionLds<kFusedWaves * kWave> sh;
  const int layer = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  for (int t = wave; t < tq; t += kFusedWaves) {
    const int64_t row = static_cast<int64_t>(layer) * tq + t;
    const int ke = select_row_wave<J, false>(score_keys + row * nblocks, nblocks, prot, nprot, k_req, order,
                                             sids + t * k_req, out_vals ? out_vals + row * k_req : nullptr,
                                             out_scores ? out_scores + row * nblocks : nullptr, pmask[wave],
                                             sel[wave], lane);
    if (t == 0 && lane == 0) s_keff = ke;   // the same for every row: one protected set per layer
  }
  __syncthreads();
  const int k_eff = s_keff;
  for (int i = tid; i < tq * k_eff; i += kFusedWaves * kWave) {
    const int t = i / k_eff, j = i % k_eff;
    out_ids[(static_cast<int64_t>(layer) * tq + t) * k_req + j] = sids[t * k_req + j];
  }
  union_layer<kFusedWaves * kWave>(sids, layer, tq, k_req, k_eff, umax, out_union, out_count, out_allowed, sh, tid);
}

struct ScoreLaunch {
  const uint16_t* q;
  int64_t q_ls;
  int nq, per_query;
  const uint16_t* reps;
  int64_t reps_ls;
  int hkv, cap, nblocks, units;
  uint32_t* keys;
  const int32_t* skip_ids;
  int n_skip;
};

template <int R, int G>
void launch_score(dim3 grid, hipStream_t s, const ScoreLaunch& a) {
  hipLaunchKernelGGL((score_kernel<R, G>), grid, dim3(kScoreThreads), 0, s, a.q, a.q_ls, a.nq, a.per_query, a.reps,
                     a.reps_ls, a.hkv, a.cap, a.nblocks, a.units, a.keys, a.skip_ids, a.n_skip);
}

template <int R>
int dispatch_g(int g, dim3 grid, hipStream_t s, const ScoreLaunch& a) {
  switch (g) {
    case 1: launch_score<R, 1>(grid, s, a); return 0;
    case 2: launch_score<R, 2>(grid, s, a); return 0;
    case 4: launch_score<R, 4>(grid, s, a); return 0;
    case 8: launch_score<R, 8>(grid, s, a); return 0;
    case 16: launch_score<R, 16>(grid, s, a); return 0;
    default: return -1;
  }
}

template <bool STEP>
void launch_topk_wave(int nblocks, dim3 rows, hipStream_t s, uint32_t* keys, const int32_t* prot, int nprot, int k,
                      int order, int32_t* out_ids, float* out_vals, float* out_scores) {
  if (nblocks <= 8 * kWave)
    hipLaunchKernelGGL((topk_wave_kernel<8, STEP>), rows, dim3(kWave), 0, s, keys, nblocks, prot, nprot, k, order,
                       out_ids, out_vals, k, out_scores);
  else if (nblocks <= 16 * kWave)
    hipLaunchKernelGGL((topk_wave_kernel<16, STEP>), rows, dim3(kWave), 0, s, keys, nblocks, prot, nprot, k, order,
                       out_ids, out_vals, k, out_scores);
  else
    hipLaunchKernelGGL((topk_wave_kernel<32, STEP>), rows, dim3(kWave), 0, s, keys, nblocks, prot, nprot, k, order,
                       out_ids, out_vals, k, out_scores);
}

// Protected lists up to this length are handled inside the decode step's
// scorer (one uniform comparison per entry and block); longer ones take the
// general selection.
constexpr int kMaxStepSkip = 64;

}  // namespace
}  // namespace nkv

using namespace nkv;

namespace nkv {

int select_impl(const nkv_store* st, int layer0, int num_layers, const uint16_t* q, int64_t q_layer_stride, int nq,
                int per_query, int nblocks, const int32_t* protected_ids, int n_protected, int k, int order,
                uint32_t* score_keys, float* out_scores, int32_t* out_ids, float* out_vals, bool step,
                void* stream, const UnionOut* uo) {
  int rc = check_store(st, layer0, num_layers);
  if (rc != NKV_OK) return rc;
  NKV_CHECK_ARG(q != nullptr && score_keys != nullptr && out_ids != nullptr,
                "nkv_select: q, score_keys and out_ids must be non-NULL");
  NKV_CHECK_ARG(nq >= 1 && nq <= 64, "nkv_select: nq must be in [1, 64] (got %d)", nq);
  NKV_CHECK_ARG(nblocks >= 1, "nkv_select: selection needs at least one history block (nblocks=%d)", nblocks);
  NKV_CHECK_ARG(nblocks <= st->cap_blocks, "nkv_select: nblocks %d exceeds cap_blocks %d", nblocks, st->cap_blocks);
  NKV_CHECK_SUPPORTED(nblocks <= kMaxSelectBlocks, "nkv_select: nblocks %d exceeds %d", nblocks, kMaxSelectBlocks);
  NKV_CHECK_ARG(k >= 1 && k <= kMaxTopk, "nkv_select: k must be in [1, %d] (got %d)", kMaxTopk, k);
  NKV_CHECK_ARG(n_protected >= 0 && (n_protected == 0 || protected_ids != nullptr),
                "nkv_select: protected list is NULL but n_protected=%d", n_protected);
  NKV_CHECK_ARG(order == NKV_ORDER_SCORE_DESC || order == NKV_ORDER_ID_ASC, "nkv_select: unknown order %d", order);
  NKV_CHECK_ARG(q_layer_stride >= static_cast<int64_t>(nq) * st->num_heads * kHeadDim || num_layers == 1,
                "nkv_select: q_layer_stride too small");
  // the decode step's form: one query, no raw scores / values, a short
  // protected list, rows the wave top-k covers
  step = step && nq == 1 && !per_query && out_scores == nullptr && out_vals == nullptr &&
         n_protected <= kMaxStepSkip && nblocks <= 32 * kWave;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int g = st->num_heads / st->num_kv_heads;
  const int R = st->r;
  const int TB = kWave / R;
  const int nqo = per_query ? nq : 1;
  ScoreLaunch a;
  a.q = q;
  a.q_ls = q_layer_stride;
  a.nq = nq;
  a.per_query = per_query;
  a.reps_ls = static_cast<int64_t>(st->num_kv_heads) * st->cap_blocks * R * kHeadDim;
  a.reps = static_cast<const uint16_t*>(st->reps) + layer0 * a.reps_ls;
  a.hkv = st->num_kv_heads;
  a.cap = st->cap_blocks;
  a.nblocks = nblocks;
  a.units = ((nblocks + TB - 1) / TB) * st->num_kv_heads;
  a.keys = score_keys;
  a.skip_ids = step ? protected_ids : nullptr;
  a.n_skip = step ? n_protected : 0;
  const bool pow2 = (g & (g - 1)) == 0 && g <= 16 && (R & (R - 1)) == 0 && R <= 8;
  NKV_CHECK_SUPPORTED(pow2, "nkv_select: unsupported (r=%d, G=%d)", R, g);
  int bad = 0;
  if (nq >= 2 && nq * g >= 2 * kScoreWaves) {
    // several queries: the workgroup-per-tile form, QB query rows per pass
    const int per = (nq * g + kScoreWaves - 1) / kScoreWaves;
    const int log_g = __builtin_ctz(g), log_r = __builtin_ctz(R);
    const dim3 grid(((nblocks + 2 * TB - 1) / (2 * TB)) * st->num_kv_heads, num_layers);  // 128 rows each
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, dim3(kScoreThreads), 0, s, a.q, a.q_ls, a.nq, a.per_query, log_g, a.reps,
                         a.reps_ls, a.hkv, a.cap, a.nblocks, log_r, a.keys);
    };
    // the pass width (2, 4 or 6 rows) that repeats the fewest rows in the
    // last group, the wider on ties (8 rows would spill scalar registers)
    int qb = 6;
    for (const int w : {4, 2})
      if ((per + w - 1) / w * w < (per + qb - 1) / qb * qb) qb = w;
    if (qb == 2) go(score_multi_kernel<2, kScoreQLds>);
    else if (qb == 4) go(score_multi_kernel<4, kScoreQLds>);
    else go(score_multi_kernel<6, kScoreQLds>);
  } else {
    dim3 grid(((a.units / st->num_kv_heads + kScoreWaves - 1) / kScoreWaves) * st->num_kv_heads, num_layers);
    switch (R) {
      case 1: bad = dispatch_g<1>(g, grid, s, a); break;
      case 2: bad = dispatch_g<2>(g, grid, s, a); break;
      case 4: bad = dispatch_g<4>(g, grid, s, a); break;
      case 8: bad = dispatch_g<8>(g, grid, s, a); break;
      default: bad = -1;
    }
  }
  NKV_CHECK_SUPPORTED(bad == 0, "nkv_select: unsupported (r=%d, G=%d)", R, g);
  rc = launch_status("nkv_select/score");
  if (rc != NKV_OK) return rc;

  if (uo != nullptr) {
    NKV_CHECK_SUPPORTED(per_query && nq <= kFusedMaxQ && k <= kFusedMaxK && nblocks <= 32 * kWave,
                        "nkv_select_per_query: needs nq <= %d, k <= %d and nblocks <= %d (got %d, %d, %d)",
                        kFusedMaxQ, kFusedMaxK, 32 * kWave, nq, k, nblocks);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(num_layers), dim3(kFusedWaves * kWave), 0, s, score_keys, nblocks, protected_ids,
                         n_protected, k, nq, order, out_ids, out_vals, out_scores, uo->umax, uo->out_union,
                         uo->out_count, uo->out_allowed);
    };
    if (nblocks <= 8 * kWave) go(topk_union_kernel<8>);
    else if (nblocks <= 16 * kWave) go(topk_union_kernel<16>);
    else go(topk_union_kernel<32>);
    return launch_status("nkv_select_per_query/topk+union");
  }
  const dim3 rows(num_layers * nqo);
  if (step) {
    launch_topk_wave<true>(nblocks, rows, s, score_keys, nullptr, 0, k, order, out_ids, nullptr, nullptr);
    return launch_status("nkv_select/topk");
  }
  if (nblocks <= 32 * kWave) {
    launch_topk_wave<false>(nblocks, rows, s, score_keys, protected_ids, n_protected, k, order, out_ids, out_vals,
                            out_scores);
    return launch_status("nkv_select/topk");
  }
  const int nwords = (nblocks + 31) >> 5;
  const size_t tsmem = static_cast<size_t>(nblocks + nwords) * sizeof(uint32_t);
  hipLaunchKernelGGL(topk_kernel, rows, dim3(kTopkThreads), tsmem, s, score_keys,
                     nblocks, protected_ids, n_protected, k, order, out_ids, out_vals, k, out_scores);
  return launch_status("nkv_select/topk");
}

bool select_step_form(int nq, int n_protected, int nblocks) {
  return nq == 1 && n_protected <= kMaxStepSkip && nblocks <= 32 * kWave;
}

}  // namespace nkv

extern "C" int nkv_select(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                          int64_t q_layer_stride, int nq, int per_query, int nblocks,
                          const int32_t* protected_ids, int n_protected, int k, int order,
                          uint32_t* score_keys, float* out_scores, int32_t* out_ids,
                          float* out_vals, void* stream) {
  return select_impl(st, layer0, num_layers, q, q_layer_stride, nq, per_query, nblocks, protected_ids, n_protected,
                     k, order, score_keys, out_scores, out_ids, out_vals, false, stream);
}

extern "C" int nkv_select_per_query(const nkv_store* st, int layer0, int num_layers, const uint16_t* q,
                                    int64_t q_layer_stride, int nq, int nblocks, const int32_t* protected_ids,
                                    int n_protected, int k, uint32_t* score_keys, float* out_scores,
                                    int32_t* out_ids, float* out_vals, int umax, int32_t* out_union,
                                    int32_t* out_count, uint8_t* out_allowed, void* stream) {
  NKV_CHECK_ARG(out_union != nullptr && out_count != nullptr && out_allowed != nullptr,
                "nkv_select_per_query: out_union, out_count and out_allowed must be non-NULL");
  NKV_CHECK_ARG(nq >= 1 && nq <= kFusedMaxQ, "nkv_select_per_query: nq must be in [1, %d] (got %d)", kFusedMaxQ, nq);
  NKV_CHECK_ARG(k >= 1 && k <= kFusedMaxK, "nkv_select_per_query: k must be in [1, %d] (got %d)", kFusedMaxK, k);
  NKV_CHECK_ARG(nblocks >= 1, "nkv_select_per_query: selection needs at least one history block (nblocks=%d)",
                nblocks);
  NKV_CHECK_SUPPORTED(nblocks <= 32 * kWave, "nkv_select_per_query: nblocks %d exceeds %d", nblocks, 32 * kWave);
  const int kmax = k < nblocks ? k : nblocks;   // bounds every row's selection
  NKV_CHECK_ARG(umax >= nq * kmax, "nkv_select_per_query: umax %d < nq * min(k, nblocks) = %d", umax, nq * kmax);
  const UnionOut uo{umax, out_union, out_count, out_allowed};
  return select_impl(st, layer0, num_layers, q, q_layer_stride, nq, 1, nblocks, protected_ids, n_protected, k,
                     NKV_ORDER_SCORE_DESC, score_keys, out_scores, out_ids, out_vals, false, stream, &uo);
}

extern "C" int nkv_select_union(const int32_t* ids, int num_layers, int tq, int k, int k_eff, int umax,
                                int32_t* out_union, int32_t* out_count, uint8_t* out_allowed, void* stream) {
  NKV_CHECK_ARG(ids != nullptr && out_union != nullptr && out_count != nullptr && out_allowed != nullptr,
                "nkv_select_union: ids, out_union, out_count and out_allowed must be non-NULL");
  NKV_CHECK_ARG(num_layers >= 1, "nkv_select_union: num_layers must be >= 1 (got %d)", num_layers);
  NKV_CHECK_ARG(tq >= 1 && tq <= 16, "nkv_select_union: tq must be in [1, 16] (got %d)", tq);
  NKV_CHECK_ARG(k_eff >= 1 && k_eff <= k, "nkv_select_union: k_eff must be in [1, k] (got %d, k=%d)", k_eff, k);
  NKV_CHECK_SUPPORTED(tq * k_eff <= kUnionMax, "nkv_select_union: tq * k_eff = %d exceeds %d", tq * k_eff,
                      kUnionMax);
  NKV_CHECK_ARG(umax >= tq * k_eff, "nkv_select_union: umax %d < tq * k_eff = %d", umax, tq * k_eff);
  hipLaunchKernelGGL(union_kernel, dim3(num_layers), dim3(kUnionThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     ids, tq, k, k_eff, umax, out_union, out_count, out_allowed);
  return launch_status("nkv_select_union");
}
