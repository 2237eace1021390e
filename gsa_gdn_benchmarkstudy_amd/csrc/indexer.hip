// Gated lightning indexer on gfx950 MFMA, and its fused exact top-k select.
//
//   S[b,i,j] = sum_h sigmoid(w[b,i,h]) * sigmoid(scale*<q[b,i,h,:], k[b,j,:]> + bias[h])
//
// (semantics of gsa_triton/gsa_ref.py:97-126).  Both kernels below share one
// score routine -- the same MFMA sequence and the same epilogue instructions
// -- so a score is bit-identical wherever it is computed; the fused selector
// relies on that to recompute scores pass after pass.
//
// Tiling: one wave owns 16 query rows.  Its MFMA A operand (q, 4 heads x 64
// dims) stays in registers for the whole kernel; keys stream through in tiles
// of 16, each tile one 16x16 output block per head:
//   bf16: v_mfma_f32_16x16x32_bf16, 2 k-steps per head  (8 MFMA per tile)
//   fp32: v_mfma_f32_16x16x4_f32,  16 k-steps per head (64 MFMA per tile)
// Output layout of a 16x16 block: lane l holds rows 4*(l/16)+e (e = 0..3) of
// column l%16.
#include "gsa_common.h"

#pragma clang fp contract(off)

namespace gsa {

constexpr int kHi = 4;    // indexer heads
constexpr int kDi = 64;   // indexer head dim

template <typename T> struct Mfma;

template <> struct Mfma<uint16_t> {
  static constexpr int kSteps = 2;          // 64 dims / 32 per MFMA
  typedef bf16x8 Op;
  // lane group g = lane/16 supplies k = 32*s + 8*g .. +7 of its row/column
  __device__ static Op load(const uint16_t* rowp, int off, int s, int g) {
    return *reinterpret_cast<const bf16x8*>(rowp + off + s * 32 + g * 8);
  }
  __device__ static floatx4 mma(Op a, Op b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  static constexpr int kSteps = 16;         // 64 dims / 4 per MFMA
  typedef float Op;
  __device__ static Op load(const float* rowp, int off, int s, int g) {
    return rowp[off + s * 4 + g];
  }
  __device__ static floatx4 mma(Op a, Op b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

struct IdxArgs {
  const void* q; int64_t q_sb, q_st;
  const void* k; int64_t k_sb, k_st;
  const void* w; int64_t w_sb, w_st;
  const float* bias;    // device fp32 [Hi]
  float scale_l2;       // -scale * log2(e)
  int B, T;
};

// Per-lane state of one wave's 16-row group.
template <typename T>
struct RowGroup {
  typename Mfma<T>::Op qa[kHi][Mfma<T>::kSteps];  // A operand: row r0 + lane%16
  float a[4][kHi];                                // sigmoid(w) of rows r0 + 4*(lane/16) + e
  float bias_l2[kHi];                             // -bias[h] * log2(e)
  float scale_l2;                                 // -scale * log2(e)
  const T* kbase;                                 // k_idx of this batch
  int64_t k_st;

  __device__ void init(const IdxArgs& p, int b, int r0, int lane) {
    const int g = lane >> 4, lr = lane & 15;
    const T* qb = static_cast<const T*>(p.q) + b * p.q_sb;
    const int qrow = min(r0 + lr, p.T - 1);
    const T* qrp = qb + (int64_t)qrow * p.q_st;
#pragma unroll
    for (int h = 0; h < kHi; ++h)
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) qa[h][s] = Mfma<T>::load(qrp, h * kDi, s, g);
    const T* wb = static_cast<const T*>(p.w) + b * p.w_sb;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = min(r0 + 4 * g + e, p.T - 1);
#pragma unroll
      for (int h = 0; h < kHi; ++h) {
        const T wv = wb[(int64_t)row * p.w_st + h];
        float wf;
        if constexpr (Elem<T>::kBf16) wf = __uint_as_float((uint32_t)wv << 16);
        else wf = wv;
        a[e][h] = sigmoidf_fast(wf);
      }
    }
    kbase = static_cast<const T*>(p.k) + b * p.k_sb;
    k_st = p.k_st;
#pragma unroll
    for (int h = 0; h < kHi; ++h) bias_l2[h] = -p.bias[h] * kLog2e;
    scale_l2 = p.scale_l2;
  }

  // B operand of key tile [j0, j0+16): column lane%16, clamped to a valid row.
  __device__ void load_keys(int j0, int T_, int lane, typename Mfma<T>::Op (&kb)[Mfma<T>::kSteps]) const {
    const int j = min(j0 + (lane & 15), T_ - 1);
    const T* krp = kbase + (int64_t)j * k_st;
#pragma unroll
    for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = Mfma<T>::load(krp, 0, s, lane >> 4);
  }

  __device__ void mma(const typename Mfma<T>::Op (&kb)[Mfma<T>::kSteps], floatx4 (&acc)[kHi]) const {
#pragma unroll
    for (int h = 0; h < kHi; ++h) {
      floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) c = Mfma<T>::mma(qa[h][s], kb[s], c);
      acc[h] = c;
    }
  }

  // Fused epilogue for output slot e: sum_h a_h * sigmoid(scale*dot_h + bias_h).
  __device__ float score(const floatx4 (&acc)[kHi], int e) const {
    float s = 0.f;
#pragma unroll
    for (int h = 0; h < kHi; ++h) {
      const float t = __builtin_fmaf(acc[h][e], scale_l2, bias_l2[h]);
      const float r = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
      s = (h == 0) ? a[e][h] * r : __builtin_fmaf(a[e][h], r, s);
    }
    return s;
  }
};

// ---------------------------------------------------------------------------
// Full score matrix (the fused_gated_indexer API).  4 waves per block, one
// 16-row group per wave; causal tiles above the diagonal are filled with -inf
// without computing them.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void indexer_scores_kernel(IdxArgs p, int causal, float* S,
                                                             int64_t s_sb, int64_t s_st) {
  const int lane = threadIdx.x & 63;
  const int ngroups = (p.T + 15) >> 4;
  const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= p.B * ngroups) return;
  const int b = wv / ngroups;
  const int r0 = (wv % ngroups) * 16;
  const int g = lane >> 4, lr = lane & 15;

  RowGroup<T> rg;
  rg.init(p, b, r0, lane);
  float* Sb = S + b * s_sb;

  const int jend = causal ? min(p.T, r0 + 16) : p.T;
  typename Mfma<T>::Op kb[Mfma<T>::kSteps], kn[Mfma<T>::kSteps];
  rg.load_keys(0, p.T, lane, kn);
  for (int j0 = 0; j0 < jend; j0 += 16) {
#pragma unroll
    for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = kn[s];
    if (j0 + 16 < jend) rg.load_keys(j0 + 16, p.T, lane, kn);
    floatx4 acc[kHi];
    rg.mma(kb, acc);
    const int col = j0 + lr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = r0 + 4 * g + e;
      if (row < p.T && col < p.T) {
        const float sc = (causal && col > row) ? -__builtin_inff() : rg.score(acc, e);
        Sb[(int64_t)row * s_st + col] = sc;
      }
    }
  }
  for (int j0 = ((jend + 15) >> 4) << 4; j0 < p.T; j0 += 16) {
    const int col = j0 + lr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = r0 + 4 * g + e;
      if (row < p.T && col < p.T) Sb[(int64_t)row * s_st + col] = -__builtin_inff();
    }
  }
}

// ---------------------------------------------------------------------------
// Fused indexer + exact top-k (never stores the score matrix).
//
// Output: the selection as a bitmask, bits[b][t] bit j set iff key j is one
// of row t's selected keys (W = 2*ceil(T/64) uint32 words per row; words past
// row t's causal range are zero).  One 256-thread block per 16-row group,
// heaviest groups first; its 4 waves take the group's causal 16-key tiles
// round-robin and share the row state in LDS.  Rows with t+1 <= k select
// every causal key.  For the others the scores are computed twice:
//   pass 1  value-linear histogram, bin = floor(s * NB / sum_h sigmoid(w_h))
//           -> the bin b1 holding the k-th largest score and the rank of the
//           k-th largest inside it;
//   pass 2  entries in bins above b1 are selected: ballot -> one 16-bit chunk
//           of the row's bitmask per 16-key tile; entries in b1 (at most
//           kCap per row) are collected as (key, index);
//   resolve exact MSB-first radix select among a row's candidates -> the
//           threshold key theta and how many entries equal to theta to take,
//           lowest indices first; winning candidates are OR-ed into the mask.
// A bin holding more than kCap entries (degenerate scores, e.g. all equal)
// falls back to four 8-bit radix passes over the bin, then one ordered pass
// by a single wave marks the winners.
// ---------------------------------------------------------------------------
constexpr int kNB = 512;                 // histogram bins per row
constexpr int kCap = 512;                // candidates per row
constexpr int kHStride = kNB + 1;        // odd stride: one bin of 16 rows in distinct banks
constexpr int kGroupWaves = 4;

enum RowMode : int { kNone = 0, kTrivial = 1, kActive = 2, kResolved = 3, kOverflow = 4 };

__device__ __forceinline__ int bin_of(float s, float inv_w) {
  return (int)fmaxf(0.f, fminf(s * inv_w, (float)(kNB - 1)));
}

// Causal-prefix chunk of row `row` for 16-key tile `tile`: keys <= row set.
__device__ __forceinline__ uint16_t prefix_chunk(int row, int tile) {
  const int n = row - 16 * tile + 1;    // keys of this tile at or before the row
  return n >= 16 ? (uint16_t)0xffffu : (n <= 0 ? (uint16_t)0 : (uint16_t)((1u << n) - 1u));
}

template <typename T>
__global__ __launch_bounds__(256) void indexer_bits_kernel(IdxArgs p, int k_eff, uint32_t* bits,
                                                           int64_t b_sb, int64_t b_st) {
  __shared__ uint32_t sh[16 * kHStride];   // histogram, then candidate keys
  __shared__ uint32_t sh_idx[16 * kCap];   // candidate key indices
  __shared__ uint32_t sh_cnt[16];
  __shared__ int st_mode[16], st_b1[16], st_need[16];
  __shared__ uint32_t st_key[16];
  __shared__ int st_any[2];                // [0] any active row, [1] any overflow

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int ngroups = (p.T + 15) >> 4;
  const int b = blockIdx.x % p.B;
  const int rg_idx = ngroups - 1 - blockIdx.x / p.B;
  const int r0 = rg_idx * 16;
  uint32_t* bbase = bits + b * b_sb;
  uint16_t* b16 = reinterpret_cast<uint16_t*>(bbase);
  const int64_t row16 = 2 * b_st;          // uint16 chunks per row

  if (tid < 16) {
    const int row = r0 + tid;
    st_mode[tid] = row >= p.T ? kNone : (row + 1 > k_eff ? kActive : kTrivial);
    st_need[tid] = k_eff;
    sh_cnt[tid] = 0u;
  }
  if (tid < 2) st_any[tid] = 0;
  __syncthreads();
  if (tid < 16 && st_mode[tid] == kActive) st_any[0] = 1;

  // Every chunk after the diagonal tile is zero; trivial rows get their
  // causal prefix now.  (The zeroing is largest for the lightest groups.)
  const int ntl = rg_idx + 1;                  // causal 16-key tiles 0 .. rg_idx
  const int zend = (rg_idx | 3) + 1;           // chunks up to the end of the 64-key tile
  for (int i = tid; i < 16 * zend; i += 256) {
    const int rl = i / zend, tile = i % zend;
    const int row = r0 + rl;
    if (row >= p.T) continue;
    if (tile >= ntl) b16[row * row16 + tile] = 0;
    else if (st_mode[rl] == kTrivial) b16[row * row16 + tile] = prefix_chunk(row, tile);
  }
  {
    const int W = 2 * ((p.T + 63) >> 6);
    const int d0 = zend >> 2;                    // first 8-byte pair of words past the 64-key tile
    const int npair = (W >> 1) - d0;
    for (int i = tid; i < 16 * npair; i += 256) {
      const int rl = i / npair, pr = d0 + i % npair;
      const int row = r0 + rl;
      if (row < p.T) reinterpret_cast<uint2*>(bbase + (int64_t)row * b_st)[pr] = uint2{0u, 0u};
    }
  }
  __syncthreads();
  if (!st_any[0]) return;

  RowGroup<T> rgp;
  rgp.init(p, b, r0, lane);
  int mode[4], b1[4];
  float inv_w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mode[e] = st_mode[4 * g + e];
    const float smax = ((rgp.a[e][0] + rgp.a[e][1]) + rgp.a[e][2]) + rgp.a[e][3];
    inv_w[e] = (float)kNB / (smax * 1.0009765625f + 1e-30f);
    b1[e] = 0;
  }

  typename Mfma<T>::Op kb[Mfma<T>::kSteps], kn[Mfma<T>::kSteps];
  // This wave's tiles: wave, wave+4, ...; f(e, row, col, tile, valid, score).
  auto sweep = [&](auto&& f) {
    int t = wave;
    if (t < ntl) rgp.load_keys(t * 16, p.T, lane, kn);
    for (; t < ntl; t += kGroupWaves) {
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = kn[s];
      if (t + kGroupWaves < ntl) rgp.load_keys((t + kGroupWaves) * 16, p.T, lane, kn);
      floatx4 acc[kHi];
      rgp.mma(kb, acc);
      const int col = t * 16 + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + 4 * g + e;
        const bool valid = mode[e] == kActive && col <= row;
        f(e, row, col, t, valid, valid ? rgp.score(acc, e) : 0.f);
      }
    }
  };

  auto scan_row = [&](int rl, int& nd) -> int {     // top-down cumulative search
    int cum = 0, bsel = 0;
    for (int bin = kNB - 1; bin >= 0; --bin) {
      const int c = (int)sh[rl * kHStride + bin];
      if (cum + c >= nd) { bsel = bin; break; }
      cum += c;
    }
    nd -= cum;
    return bsel;
  };
  auto zero_hist = [&]() {
    for (int i = tid; i < 16 * kHStride; i += 256) sh[i] = 0u;
    __syncthreads();
  };

  // ---- pass 1: histogram ---------------------------------------------------
  zero_hist();
  sweep([&](int e, int, int, int, bool valid, float s) {
    if (valid) atomicAdd(&sh[(4 * g + e) * kHStride + bin_of(s, inv_w[e])], 1u);
  });
  __syncthreads();
  if (tid < 16 && st_mode[tid] == kActive) {
    int nd = st_need[tid];
    st_b1[tid] = scan_row(tid, nd);
    st_need[tid] = nd;
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; ++e) b1[e] = st_b1[4 * g + e];
  __syncthreads();   // sh is reused for candidate keys below

  // ---- pass 2: bins above b1 -> mask chunks; bin b1 -> candidates ------------
  sweep([&](int e, int row, int col, int t, bool valid, float s) {
    const int bn = bin_of(s, inv_w[e]);
    const bool sel = valid && bn > b1[e];
    if (valid && bn == b1[e]) {
      const int rl = 4 * g + e;
      const uint32_t pos = atomicAdd(&sh_cnt[rl], 1u);
      if (pos < (uint32_t)kCap) {
        sh[rl * kHStride + pos] = score_key(s);
        sh_idx[rl * kCap + pos] = (uint32_t)col;
      }
    }
    const uint64_t m = ballot64(sel);
    if (lr == 0 && mode[e] == kActive) b16[row * row16 + t] = (uint16_t)(m >> (16 * g));
  });
  __threadfence();
  __syncthreads();

  // ---- resolve: wave w takes rows 4w .. 4w+3 ----------------------------------
  for (int q = 0; q < 4; ++q) {
    const int rl = 4 * wave + q;
    if (st_mode[rl] != kActive) continue;
    const int n = (int)sh_cnt[rl];
    if (n > kCap) {
      if (lane == 0) { st_mode[rl] = kOverflow; st_any[1] = 1; }
      continue;
    }
    uint32_t cv[kCap / 64], ci[kCap / 64];
#pragma unroll
    for (int i = 0; i < kCap / 64; ++i) {
      const int c = i * 64 + lane;
      cv[i] = c < n ? sh[rl * kHStride + c] : 0u;
      ci[i] = c < n ? sh_idx[rl * kCap + c] : 0u;
    }
    int k = st_need[rl];
    uint32_t prefix = 0u, pmask = 0u;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t tm = pmask | (1u << bit), tv = prefix | (1u << bit);
      int c = 0;
#pragma unroll
      for (int i = 0; i < kCap / 64; ++i) c += __popcll(ballot64((i * 64 + lane) < n && (cv[i] & tm) == tv));
      if (c >= k) prefix = tv; else k -= c;
      pmask = tm;
    }
    // winners: key > theta, or key == theta among the k lowest indices of the ties
    const int row = r0 + rl;
    uint32_t* brow = bbase + (int64_t)row * b_st;
#pragma unroll
    for (int i = 0; i < kCap / 64; ++i) {
      const int c = i * 64 + lane;
      if (c >= n) continue;
      bool win = cv[i] > prefix;
      if (cv[i] == prefix) {
        int rank = 0;
        for (int o = 0; o < n; ++o)
          rank += (sh[rl * kHStride + o] == prefix && sh_idx[rl * kCap + o] < ci[i]) ? 1 : 0;
        win = rank < k;
      }
      if (win) atomicOr(&brow[ci[i] >> 5], 1u << (ci[i] & 31));
    }
  }
  __syncthreads();
  if (!st_any[1]) return;

  // ---- overflow rows: radix passes over the keys of bin b1 --------------------
  if (tid < 16 && st_mode[tid] == kOverflow) st_key[tid] = 0u;
#pragma unroll
  for (int e = 0; e < 4; ++e) mode[e] = st_mode[4 * g + e] == kOverflow ? kActive : kNone;
  for (int level = 0; level < 4; ++level) {
    uint32_t pre[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) pre[e] = st_key[4 * g + e];
    const int hi_shift = 32 - 8 * level, lo_shift = 24 - 8 * level;
    zero_hist();
    sweep([&](int e, int, int, int, bool valid, float s) {
      if (valid && bin_of(s, inv_w[e]) == b1[e]) {
        const uint32_t key = score_key(s);
        if (level == 0 || (key >> hi_shift) == pre[e])
          atomicAdd(&sh[(4 * g + e) * kHStride + ((key >> lo_shift) & 255u)], 1u);
      }
    });
    __syncthreads();
    if (tid < 16 && st_mode[tid] == kOverflow) {
      int cum = 0, d = 0, nd = st_need[tid];
      for (int bin = 255; bin >= 0; --bin) {
        const int c = (int)sh[tid * kHStride + bin];
        if (cum + c >= nd) { d = bin; break; }
        cum += c;
      }
      st_need[tid] = nd - cum;
      st_key[tid] = (st_key[tid] << 8) | (uint32_t)d;
    }
    __syncthreads();
  }
  // wave 0 marks the winners of the overflow rows in key order (tie ranks need order)
  if (wave == 0) {
    uint32_t theta[4];
    int tie_need[4], tie_seen[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      theta[e] = st_key[4 * g + e];
      tie_need[e] = st_need[4 * g + e];
      tie_seen[e] = 0;
    }
    const uint64_t gmask = 0xffffull << (16 * g);
    rgp.load_keys(0, p.T, lane, kn);
    for (int t = 0; t < ntl; ++t) {
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = kn[s];
      if (t + 1 < ntl) rgp.load_keys((t + 1) * 16, p.T, lane, kn);
      floatx4 acc[kHi];
      rgp.mma(kb, acc);
      const int col = t * 16 + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + 4 * g + e;
        const bool valid = mode[e] == kActive && col <= row;
        const float s = valid ? rgp.score(acc, e) : 0.f;
        const bool inbin = valid && bin_of(s, inv_w[e]) == b1[e];
        const uint32_t key = score_key(s);
        const bool tie = inbin && key == theta[e];
        const uint64_t tmask = ballot64(tie) & gmask;
        const int trank = tie_seen[e] + count_below(tmask);
        tie_seen[e] += __popcll(tmask);
        if (inbin && (key > theta[e] || (tie && trank < tie_need[e])))
          atomicOr(&bbase[(int64_t)row * b_st + (col >> 5)], 1u << (col & 31));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Bitmask -> ascending indices + count, one 256-thread block per row.  The
// tail of a row with fewer than k selected keys is t+1, t+2, ... (the
// lowest-index invalid entries, as the selector orders them).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void bits_to_indices_kernel(const uint32_t* __restrict__ bits, int64_t b_sb,
                                                              int64_t b_st, int T, int W, int k_eff,
                                                              int32_t* __restrict__ idx_out,
                                                              int32_t* __restrict__ count_out) {
  __shared__ int wave_tot[4];
  const int row = blockIdx.x;
  const int b = row / T, t = row % T;
  const uint32_t* brow = bits + b * b_sb + (int64_t)t * b_st;
  int32_t* orow = idx_out + (int64_t)row * k_eff;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (W + 255) / 256;       // contiguous words per thread
  const int w0 = min(W, tid * per), w1 = min(W, w0 + per);
  int cnt = 0;
  for (int wd = w0; wd < w1; ++wd) cnt += __popc(brow[wd]);
  // exclusive prefix over the block
  int incl = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int base = incl - cnt, total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (w < wave) base += wave_tot[w];
    total += wave_tot[w];
  }
  int pos = base;
  for (int wd = w0; wd < w1; ++wd) {
    uint32_t m = brow[wd];
    while (m) {
      const int bit = __ffs(m) - 1;
      m &= m - 1;
      if (pos < k_eff) orow[pos] = wd * 32 + bit;
      ++pos;
    }
  }
  const int n = min(total, k_eff);
  for (int i = n + tid; i < k_eff; i += 256) orow[i] = t + 1 + (i - n);
  if (tid == 0) count_out[row] = n;
}

}  // namespace gsa

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
using namespace gsa_host;

static int check_indexer_args(const void* q, int64_t q_sb, int64_t q_st, const void* k, int64_t k_sb,
                              int64_t k_st, const void* w, const float* bias, int B, int T, int Hi,
                              int di, int dtype) {
  if (!q || !k || !w || !bias) return GSA_ERR_NULL;
  if (dtype_size(dtype) == 0) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || Hi != gsa::kHi || di != gsa::kDi) return GSA_ERR_SHAPE;
  if (!vec_ok(q, q_sb, q_st, dtype) || !vec_ok(k, k_sb, k_st, dtype)) return GSA_ERR_ALIGN;
  if (!aligned(w, dtype_size(dtype)) || !aligned(bias, 4)) return GSA_ERR_ALIGN;
  return GSA_OK;
}

static gsa::IdxArgs make_idx_args(const void* q, int64_t q_sb, int64_t q_st, const void* k, int64_t k_sb,
                                  int64_t k_st, const void* w, int64_t w_sb, int64_t w_st,
                                  const float* bias, float scale, int B, int T) {
  gsa::IdxArgs a;
  a.q = q; a.q_sb = q_sb; a.q_st = q_st;
  a.k = k; a.k_sb = k_sb; a.k_st = k_st;
  a.w = w; a.w_sb = w_sb; a.w_st = w_st;
  a.bias = bias;
  a.scale_l2 = -scale * gsa::kLog2e;
  a.B = B; a.T = T;
  return a;
}

extern "C" int gsa_indexer_scores(const void* q_idx, int64_t q_sb, int64_t q_st,
                                  const void* k_idx, int64_t k_sb, int64_t k_st,
                                  const void* w, int64_t w_sb, int64_t w_st,
                                  const float* bias, float scale,
                                  int B, int T, int Hi, int di, int causal, int dtype,
                                  float* scores, int64_t s_sb, int64_t s_st,
                                  void* stream) {
  int st = check_indexer_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype);
  if (st) return st;
  if (!scores) return GSA_ERR_NULL;
  if (!aligned(scores, 4)) return GSA_ERR_ALIGN;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  const int ngroups = (T + 15) / 16;
  const int waves = B * ngroups;
  dim3 grid((waves + 3) / 4), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GSA_DTYPE_BF16)
    hipLaunchKernelGGL(gsa::indexer_scores_kernel<uint16_t>, grid, block, 0, s, a, causal, scores, s_sb, s_st);
  else
    hipLaunchKernelGGL(gsa::indexer_scores_kernel<float>, grid, block, 0, s, a, causal, scores, s_sb, s_st);
  return launch_status();
}

extern "C" int gsa_indexer_select(const void* q_idx, int64_t q_sb, int64_t q_st,
                                  const void* k_idx, int64_t k_sb, int64_t k_st,
                                  const void* w, int64_t w_sb, int64_t w_st,
                                  const float* bias, float scale,
                                  int B, int T, int Hi, int di, int k_eff, int dtype,
                                  uint32_t* bits, int64_t b_sb, int64_t b_st,
                                  int32_t* idx_out, int32_t* count_out,
                                  void* stream) {
  int st = check_indexer_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype);
  if (st) return st;
  if (!bits) return GSA_ERR_NULL;
  if ((idx_out == nullptr) != (count_out == nullptr)) return GSA_ERR_NULL;
  if (k_eff < 1 || k_eff > T) return GSA_ERR_K;
  const int W = 2 * ((T + 63) / 64);
  if (b_st < W || (B > 1 && b_sb < (int64_t)T * b_st)) return GSA_ERR_SHAPE;
  if (!aligned(bits, 8) || (b_st % 2) || (b_sb % 2)) return GSA_ERR_ALIGN;
  if (idx_out && (!aligned(idx_out, 4) || !aligned(count_out, 4))) return GSA_ERR_ALIGN;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  const int ngroups = (T + 15) / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GSA_DTYPE_BF16)
    hipLaunchKernelGGL(gsa::indexer_bits_kernel<uint16_t>, dim3(B * ngroups), dim3(256), 0, s, a, k_eff, bits,
                       b_sb, b_st);
  else
    hipLaunchKernelGGL(gsa::indexer_bits_kernel<float>, dim3(B * ngroups), dim3(256), 0, s, a, k_eff, bits,
                       b_sb, b_st);
  st = launch_status();
  if (st || !idx_out) return st;
  hipLaunchKernelGGL(gsa::bits_to_indices_kernel, dim3(B * T), dim3(256), 0, s, bits, b_sb, b_st, T, W, k_eff,
                     idx_out, count_out);
  return launch_status();
}
