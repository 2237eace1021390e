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
// One wave per 16-row group, heaviest groups first.  Rows with t+1 <= k
// select every causal key.  For the other rows the scores are recomputed in
// passes over the causal key tiles:
//   1. HIST   histogram of value-linear bins  bin = floor(s * NB / sum_h a_h)
//             -> the bin b1 holding the k-th largest score, and how many of
//             the bin's entries are still needed.
//   2. COLLECT keys of the entries in bin b1 (at most kCap) -> exact radix
//             select among them -> threshold key theta and the number of
//             entries equal to theta to take (lowest indices first).
//      DIGIT  (only when a bin overflows kCap): four 8-bit radix passes over
//             the keys in bin b1 replace COLLECT.
//   3. EMIT   entries with key > theta, plus the first tie_need entries with
//             key == theta, written in ascending key-index order.
// ---------------------------------------------------------------------------
constexpr int kNB = 256;
constexpr int kCap = 256;
constexpr int kLdsStride = kNB + 1;   // odd stride: rows of one bin in distinct banks

enum RowMode : int { kTrivial = 0, kActive = 1, kResolved = 2, kOverflow = 3 };

__device__ __forceinline__ int bin_of(float s, float inv_w) {
  return (int)fmaxf(0.f, fminf(s * inv_w, (float)(kNB - 1)));
}

template <typename T>
__global__ __launch_bounds__(64) void indexer_select_kernel(IdxArgs p, int k_eff, int32_t* idx_out,
                                                            int32_t* count_out) {
  __shared__ uint32_t sh[16 * kLdsStride];   // histogram bins, or candidate keys
  __shared__ uint32_t sh_cnt[16];
  __shared__ int st_mode[16], st_b1[16], st_need[16];
  __shared__ uint32_t st_key[16];            // radix prefix, then theta

  const int lane = threadIdx.x;
  const int g = lane >> 4, lr = lane & 15;
  const int ngroups = (p.T + 15) >> 4;
  const int b = blockIdx.x % p.B;
  const int r0 = (ngroups - 1 - blockIdx.x / p.B) * 16;
  const int64_t out_row0 = (int64_t)b * p.T;

  // Row classification (lane < 16 owns row r0 + lane).
  if (lane < 16) {
    const int row = r0 + lane;
    st_mode[lane] = (row < p.T && row + 1 > k_eff) ? kActive : kTrivial;
    st_need[lane] = k_eff;
  }
  __syncthreads();

  // Trivial rows: every causal key, then t+1, t+2, ... (the lowest-index
  // invalid entries), i.e. the row is 0..k_eff-1 with count t+1.
  bool any_active = false;
  for (int rl = 0; rl < 16; ++rl) {
    const int row = r0 + rl;
    if (row >= p.T) break;
    if (st_mode[rl] == kActive) { any_active = true; continue; }
    int32_t* orow = idx_out + (out_row0 + row) * k_eff;
    for (int m = lane; m < k_eff; m += 64) orow[m] = m;
    if (lane == 0) count_out[out_row0 + row] = row + 1;
  }
  if (!any_active) return;

  RowGroup<T> rg;
  rg.init(p, b, r0, lane);
  int mode[4], b1[4], need[4];
  float inv_w[4];
  uint32_t theta[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int rl = 4 * g + e;
    mode[e] = st_mode[rl];
    need[e] = k_eff;
    const float smax = ((rg.a[e][0] + rg.a[e][1]) + rg.a[e][2]) + rg.a[e][3];
    inv_w[e] = (float)kNB / (smax * 1.0009765625f + 1e-30f);
    b1[e] = 0;
    theta[e] = 0;
  }
  const int ntl = (r0 >> 4) + 1;   // causal key tiles 0 .. r0/16

  typename Mfma<T>::Op kb[Mfma<T>::kSteps], kn[Mfma<T>::kSteps];

  // Visit every causal (row, key) of the group; f(e, row, col, score) runs on
  // entries of active rows.
  auto sweep = [&](auto&& f) {
    rg.load_keys(0, p.T, lane, kn);
    for (int t = 0; t < ntl; ++t) {
      const int j0 = t * 16;
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = kn[s];
      if (t + 1 < ntl) rg.load_keys(j0 + 16, p.T, lane, kn);
      floatx4 acc[kHi];
      rg.mma(kb, acc);
      const int col = j0 + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + 4 * g + e;
        const bool valid = (mode[e] != kTrivial) && col <= row;   // row < T for non-trivial
        f(e, row, col, valid, valid ? rg.score(acc, e) : 0.f);
      }
    }
  };

  auto zero_sh = [&]() {
    for (int i = lane; i < 16 * kLdsStride; i += 64) sh[i] = 0u;
    if (lane < 16) sh_cnt[lane] = 0u;
    __syncthreads();
  };

  // Lane rl < 16: scan row rl's histogram from the top for the bin holding
  // the need-th largest entry.  Returns the bin; need becomes the rank
  // inside that bin.
  auto scan_row = [&](int rl, int& nd) -> int {
    int cum = 0, bsel = 0;
    for (int bin = kNB - 1; bin >= 0; --bin) {
      const int c = (int)sh[rl * kLdsStride + bin];
      if (cum + c >= nd) { bsel = bin; break; }
      cum += c;
    }
    nd -= cum;
    return bsel;
  };

  // ---- pass 1: value-linear histogram ------------------------------------
  zero_sh();
  sweep([&](int e, int, int, bool valid, float s) {
    if (valid) atomicAdd(&sh[(4 * g + e) * kLdsStride + bin_of(s, inv_w[e])], 1u);
  });
  __syncthreads();
  if (lane < 16 && st_mode[lane] == kActive) {
    int nd = st_need[lane];
    st_b1[lane] = scan_row(lane, nd);
    st_need[lane] = nd;
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; ++e) { b1[e] = st_b1[4 * g + e]; need[e] = st_need[4 * g + e]; }

  // ---- pass 2: collect the keys of bin b1 --------------------------------
  zero_sh();
  sweep([&](int e, int, int, bool valid, float s) {
    if (valid && bin_of(s, inv_w[e]) == b1[e]) {
      const int rl = 4 * g + e;
      const uint32_t pos = atomicAdd(&sh_cnt[rl], 1u);
      if (pos < (uint32_t)kCap) sh[rl * kLdsStride + pos] = score_key(s);
    }
  });
  __syncthreads();
  // Exact radix select among the candidates, one row at a time across the wave.
  bool any_overflow = false;
  for (int rl = 0; rl < 16; ++rl) {
    if (st_mode[rl] != kActive) continue;
    const int n = (int)sh_cnt[rl];
    if (n > kCap) { any_overflow = true; continue; }
    uint32_t cv[kCap / 64];
#pragma unroll
    for (int i = 0; i < kCap / 64; ++i) {
      const int idx = i * 64 + lane;
      cv[i] = idx < n ? sh[rl * kLdsStride + idx] : 0u;
    }
    int k = st_need[rl];
    uint32_t prefix = 0u, pmask = 0u;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t tm = pmask | (1u << bit), tv = prefix | (1u << bit);
      int c = 0;
#pragma unroll
      for (int i = 0; i < kCap / 64; ++i)
        c += __popcll(ballot64((i * 64 + lane) < n && (cv[i] & tm) == tv));
      if (c >= k) prefix = tv; else k -= c;
      pmask = tm;
    }
    if (lane == 0) { st_key[rl] = prefix; st_need[rl] = k; st_mode[rl] = kResolved; }
  }
  __syncthreads();

  // ---- DIGIT passes: rows whose bin overflowed ----------------------------
  if (any_overflow) {
    if (lane < 16 && st_mode[lane] == kActive) { st_mode[lane] = kOverflow; st_key[lane] = 0u; }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) { mode[e] = st_mode[4 * g + e]; need[e] = st_need[4 * g + e]; }
    for (int level = 0; level < 4; ++level) {
      uint32_t pre[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) pre[e] = st_key[4 * g + e];
      const int hi_shift = 32 - 8 * level, lo_shift = 24 - 8 * level;
      zero_sh();
      sweep([&](int e, int, int, bool valid, float s) {
        if (valid && mode[e] == kOverflow && bin_of(s, inv_w[e]) == b1[e]) {
          const uint32_t key = score_key(s);
          if (level == 0 || (key >> hi_shift) == pre[e])
            atomicAdd(&sh[(4 * g + e) * kLdsStride + ((key >> lo_shift) & 255u)], 1u);
        }
      });
      __syncthreads();
      if (lane < 16 && st_mode[lane] == kOverflow) {
        int nd = st_need[lane];
        const int d = scan_row(lane, nd);
        st_need[lane] = nd;
        st_key[lane] = (st_key[lane] << 8) | (uint32_t)d;
      }
      __syncthreads();
    }
    if (lane < 16 && st_mode[lane] == kOverflow) st_mode[lane] = kResolved;
    __syncthreads();
  }

  // ---- pass 3: ordered emission ------------------------------------------
  int tie_need[4], tie_seen[4], emitted[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mode[e] = st_mode[4 * g + e];
    theta[e] = st_key[4 * g + e];
    tie_need[e] = st_need[4 * g + e];
    tie_seen[e] = 0;
    emitted[e] = 0;
  }
  const uint64_t gmask = 0xffffull << (16 * g);
  sweep([&](int e, int row, int col, bool valid, float s) {
    const uint32_t key = score_key(s);
    const bool tie = valid && key == theta[e];
    const uint64_t tmask = ballot64(tie) & gmask;
    const int trank = tie_seen[e] + count_below(tmask);
    tie_seen[e] += __popcll(tmask);
    const bool sel = valid && (key > theta[e] || (tie && trank < tie_need[e]));
    const uint64_t smask = ballot64(sel) & gmask;
    const int pos = emitted[e] + count_below(smask);
    if (sel && pos < k_eff) idx_out[(out_row0 + row) * k_eff + pos] = col;
    emitted[e] += __popcll(smask);
  });
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = r0 + 4 * g + e;
    if (mode[e] != kTrivial && lr == 0) count_out[out_row0 + row] = emitted[e];
  }
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
                                  int32_t* idx_out, int32_t* count_out,
                                  void* stream) {
  int st = check_indexer_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype);
  if (st) return st;
  if (!idx_out || !count_out) return GSA_ERR_NULL;
  if (k_eff < 1 || k_eff > T) return GSA_ERR_K;
  if (!aligned(idx_out, 4) || !aligned(count_out, 4)) return GSA_ERR_ALIGN;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  const int ngroups = (T + 15) / 16;
  dim3 grid(B * ngroups), block(64);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GSA_DTYPE_BF16)
    hipLaunchKernelGGL(gsa::indexer_select_kernel<uint16_t>, grid, block, 0, s, a, k_eff, idx_out, count_out);
  else
    hipLaunchKernelGGL(gsa::indexer_select_kernel<float>, grid, block, 0, s, a, k_eff, idx_out, count_out);
  return launch_status();
}
