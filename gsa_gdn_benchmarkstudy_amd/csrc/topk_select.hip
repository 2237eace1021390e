// Exact per-row top-k of an fp32 score matrix (the AdaptiveTopKSelector API).
//
// One 1024-thread block per row.  Scores map to order-preserving uint32 keys
// (score_key: -inf -> -1e9, NaN above +inf).  Four 8-bit radix passes over
// the row find the k-th largest key theta and how many entries equal to theta
// are taken; ties at theta go to the lowest indices.  The selected entries are
// then written by ordered block-wide compaction:
//   GSA_ORDER_INDEX_ASC : valid entries ascending, then invalid (-inf) ones
//   GSA_ORDER_SCORE_DESC: the selection sorted by (key desc, index asc) with a
//                         bitonic sort in LDS (k <= GSA_TOPK_DESC_MAX_K)
#include "gsa_common.h"

namespace gsa {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;

struct SelShared {
  uint32_t hist[256];
  uint32_t wave_cnt[2][kSelWaves];
  uint32_t prefix;
  int need;
};

// Exclusive block-wide prefix count of two predicates over one 1024-entry
// chunk; returns this thread's ranks and the chunk totals.
__device__ __forceinline__ void block_rank2(SelShared& sm, bool p0, bool p1, int& r0, int& r1,
                                            int& tot0, int& tot1) {
  const int wave = threadIdx.x >> 6;
  const uint64_t m0 = ballot64(p0), m1 = ballot64(p1);
  if ((threadIdx.x & 63) == 0) {
    sm.wave_cnt[0][wave] = (uint32_t)__popcll(m0);
    sm.wave_cnt[1][wave] = (uint32_t)__popcll(m1);
  }
  __syncthreads();
  int b0 = 0, b1 = 0, t0 = 0, t1 = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const int c0 = (int)sm.wave_cnt[0][w], c1 = (int)sm.wave_cnt[1][w];
    if (w < wave) { b0 += c0; b1 += c1; }
    t0 += c0; t1 += c1;
  }
  r0 = b0 + count_below(m0);
  r1 = b1 + count_below(m1);
  tot0 = t0; tot1 = t1;
  __syncthreads();   // wave_cnt is reused by the next chunk
}

// Output rows are `width` entries wide.  Row r selects k = width entries, or
// k = min(k_rows[r], width) when k_rows is given; entries k .. width-1 of a
// row are then index 0 with mask 0.
__global__ __launch_bounds__(kSelThreads) void topk_select_kernel(
    const float* __restrict__ S, int64_t s_sb, int64_t s_st, int T, int Tkv, int width,
    const int32_t* __restrict__ k_rows, int order,
    int32_t* __restrict__ idx_out, int32_t* __restrict__ count_out, uint8_t* __restrict__ mask_out) {
  __shared__ SelShared sm;
  extern __shared__ uint64_t sort_buf[];   // GSA_ORDER_SCORE_DESC only

  const int row = blockIdx.x;
  const int b = row / T, t = row % T;
  const float* srow = S + b * s_sb + (int64_t)t * s_st;
  const int tid = threadIdx.x;
  const int k = k_rows ? min(k_rows[row], width) : width;

  // ---- radix select: 4 passes of 8 bits, MSB first ----
  if (tid == 0) { sm.prefix = 0u; sm.need = k; }
  for (int level = 0; level < 4; ++level) {
    for (int i = tid; i < 256; i += kSelThreads) sm.hist[i] = 0u;
    __syncthreads();
    const uint32_t pre = sm.prefix;
    const int hi_shift = 32 - 8 * level, lo_shift = 24 - 8 * level;
    for (int j = tid; j < Tkv; j += kSelThreads) {
      const uint32_t key = score_key(srow[j]);
      if (level == 0 || (key >> hi_shift) == pre) atomicAdd(&sm.hist[(key >> lo_shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      int need = sm.need, cum = 0, d = 0;
      for (int bin = 255; bin >= 0; --bin) {
        const int c = (int)sm.hist[bin];
        if (cum + c >= need) { d = bin; break; }
        cum += c;
      }
      sm.need = need - cum;
      sm.prefix = (pre << 8) | (uint32_t)d;
    }
    __syncthreads();
  }
  const uint32_t theta = sm.prefix;
  const int tie_need = sm.need;

  const int64_t obase = (int64_t)row * width;
  for (int i = k + tid; i < width; i += kSelThreads) {
    idx_out[obase + i] = 0;
    if (mask_out) mask_out[obase + i] = 0;
  }
  if (order == GSA_ORDER_INDEX_ASC) {
    // Sweep 1 writes valid selected entries, sweep 2 the invalid ones after them.
    int n_valid = 0;
    for (int sweep = 0; sweep < 2; ++sweep) {
      int ties = 0, written = 0;
      for (int j0 = 0; j0 < Tkv; j0 += kSelThreads) {
        const int j = j0 + tid;
        float s = 0.f;
        uint32_t key = 0u;
        if (j < Tkv) { s = srow[j]; key = score_key(s); }
        const bool in = j < Tkv;
        const bool tie = in && key == theta;
        int trank, dummy, ttot, dtot;
        block_rank2(sm, tie, false, trank, dummy, ttot, dtot);
        const bool sel = in && (key > theta || (tie && ties + trank < tie_need));
        const bool valid = s != -__builtin_inff();
        const bool mine = sel && (sweep == 0 ? valid : !valid);
        int pos, dummy2, ptot, dtot2;
        block_rank2(sm, mine, false, pos, dummy2, ptot, dtot2);
        const int o = n_valid * sweep + written + pos;
        if (mine && o < k) {
          idx_out[obase + o] = j;
          if (mask_out) mask_out[obase + o] = (uint8_t)(sweep == 0);
        }
        ties += ttot;
        written += ptot;
      }
      if (sweep == 0) n_valid = written;
    }
    if (tid == 0 && count_out) count_out[row] = n_valid;
  } else {
    // Gather the selection into LDS as (key << 32 | ~index), sort descending.
    int kp = 1;
    while (kp < k) kp <<= 1;
    int ties = 0, written = 0;
    for (int j0 = 0; j0 < Tkv; j0 += kSelThreads) {
      const int j = j0 + tid;
      uint32_t key = 0u;
      if (j < Tkv) key = score_key(srow[j]);
      const bool in = j < Tkv;
      const bool tie = in && key == theta;
      int trank, dummy, ttot, dtot;
      block_rank2(sm, tie, false, trank, dummy, ttot, dtot);
      const bool sel = in && (key > theta || (tie && ties + trank < tie_need));
      int pos, d2, ptot, dt2;
      block_rank2(sm, sel, false, pos, d2, ptot, dt2);
      if (sel && written + pos < kp) sort_buf[written + pos] = ((uint64_t)key << 32) | (uint64_t)(~(uint32_t)j);
      ties += ttot;
      written += ptot;
    }
    for (int i = written + tid; i < kp; i += kSelThreads) sort_buf[i] = 0ull;  // sorts last
    __syncthreads();
    // bitonic sort, descending
    for (int size = 2; size <= kp; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < kp; i += kSelThreads) {
          const int jx = i ^ stride;
          if (jx > i) {
            const uint64_t a = sort_buf[i], c = sort_buf[jx];
            const bool desc = (i & size) == 0;
            if (desc ? (a < c) : (a > c)) { sort_buf[i] = c; sort_buf[jx] = a; }
          }
        }
        __syncthreads();
      }
    }
    int nv_local = 0;
    for (int i = tid; i < k; i += kSelThreads) {
      // padding entries (key 0) never reach the first k once k are selected;
      // clamp anyway so a short selection cannot index outside the row
      const int j = max(0, min((int)(~(uint32_t)(sort_buf[i] & 0xffffffffull)), Tkv - 1));
      idx_out[obase + i] = j;
      const bool valid = srow[j] != -__builtin_inff();
      if (mask_out) mask_out[obase + i] = (uint8_t)valid;
      nv_local += valid ? 1 : 0;
    }
    if (count_out) {
      if (tid == 0) sm.need = 0;   // reused as the valid-entry total
      __syncthreads();
      if (nv_local) atomicAdd(&sm.need, nv_local);
      __syncthreads();
      if (tid == 0) count_out[row] = sm.need;
    }
  }
}

// Population variance of each row's finite (not -inf) scores, two passes
// (mean, then squared deviations) as the variance rule states it
// (gsa_explained.ipynb:577-592); a row without finite scores gets 0.
__global__ __launch_bounds__(256) void row_var_kernel(const float* __restrict__ S, int64_t s_sb, int64_t s_st,
                                                      int T, int Tkv, float* __restrict__ var) {
  __shared__ float part[4];
  __shared__ int cpart[4];
  const int row = blockIdx.x;
  const int b = row / T, t = row % T;
  const float* srow = S + b * s_sb + (int64_t)t * s_st;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float sum = 0.f;
  int cnt = 0;
  for (int j = tid; j < Tkv; j += 256) {
    const float v = srow[j];
    if (v != -__builtin_inff()) { sum += v; ++cnt; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    sum += __shfl_xor(sum, o, 64);
    cnt += __shfl_xor(cnt, o, 64);
  }
  if (lane == 0) { part[wave] = sum; cpart[wave] = cnt; }
  __syncthreads();
  const float n = (float)max(1, cpart[0] + cpart[1] + cpart[2] + cpart[3]);
  const float mean = (((part[0] + part[1]) + part[2]) + part[3]) / n;
  __syncthreads();
  float sq = 0.f;
  for (int j = tid; j < Tkv; j += 256) {
    const float v = srow[j];
    if (v != -__builtin_inff()) {
      const float d = v - mean;
      sq = __builtin_fmaf(d, d, sq);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
  if (lane == 0) part[wave] = sq;
  __syncthreads();
  if (tid == 0) var[row] = (((part[0] + part[1]) + part[2]) + part[3]) / n;
}

}  // namespace gsa

using namespace gsa_host;

extern "C" int gsa_topk_select(const float* scores, int64_t s_sb, int64_t s_st,
                               int B, int T, int Tkv, int k_eff, int order,
                               int32_t* idx_out, int32_t* count_out, uint8_t* mask_out,
                               void* stream) {
  if (!scores || !idx_out) return GSA_ERR_NULL;
  if (B < 1 || T < 1 || Tkv < 1) return GSA_ERR_SHAPE;
  if (order != GSA_ORDER_INDEX_ASC && order != GSA_ORDER_SCORE_DESC) return GSA_ERR_FLAGS;
  if (k_eff < 1 || k_eff > Tkv) return GSA_ERR_K;
  if (order == GSA_ORDER_SCORE_DESC && k_eff > GSA_TOPK_DESC_MAX_K) return GSA_ERR_K;
  if (!aligned(scores, 4) || !aligned(idx_out, 4) || (count_out && !aligned(count_out, 4)))
    return GSA_ERR_ALIGN;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  size_t dyn = 0;
  if (order == GSA_ORDER_SCORE_DESC) {
    int kp = 1;
    while (kp < k_eff) kp <<= 1;
    dyn = (size_t)kp * sizeof(uint64_t);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gsa::topk_select_kernel, dim3(B * T), dim3(gsa::kSelThreads), dyn, s, scores, s_sb,
                     s_st, T, Tkv, k_eff, nullptr, order, idx_out, count_out, mask_out);
  return launch_status();
}

extern "C" int gsa_topk_select_adaptive(const float* scores, int64_t s_sb, int64_t s_st,
                                        int B, int T, int Tkv, int k_base, int k_min, int k_max, int order,
                                        int32_t* idx_out, int32_t* count_out, uint8_t* mask_out,
                                        int32_t* k_out, float* var_out, void* stream) {
  if (!scores || !idx_out || !k_out || !var_out) return GSA_ERR_NULL;
  if (B < 1 || T < 1 || Tkv < 1) return GSA_ERR_SHAPE;
  if (order != GSA_ORDER_INDEX_ASC && order != GSA_ORDER_SCORE_DESC) return GSA_ERR_FLAGS;
  if (k_base < 1 || k_min < 1 || k_max < k_min) return GSA_ERR_K;
  const int width = k_max < Tkv ? k_max : Tkv;
  if (order == GSA_ORDER_SCORE_DESC && width > GSA_TOPK_DESC_MAX_K) return GSA_ERR_K;
  if (!aligned(scores, 4) || !aligned(idx_out, 4) || (count_out && !aligned(count_out, 4)) ||
      !aligned(k_out, 4) || !aligned(var_out, 4))
    return GSA_ERR_ALIGN;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  size_t dyn = 0;
  if (order == GSA_ORDER_SCORE_DESC) {
    int kp = 1;
    while (kp < width) kp <<= 1;
    dyn = (size_t)kp * sizeof(uint64_t);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gsa::row_var_kernel, dim3(B * T), dim3(256), 0, s, scores, s_sb, s_st, T, Tkv, var_out);
  int st = launch_status();
  if (st) return st;
  if ((st = launch_adaptive_k(var_out, B * T, k_base, k_min, k_max, width, k_out, s))) return st;
  hipLaunchKernelGGL(gsa::topk_select_kernel, dim3(B * T), dim3(gsa::kSelThreads), dyn, s, scores, s_sb,
                     s_st, T, Tkv, width, k_out, order, idx_out, count_out, mask_out);
  return launch_status();
}
