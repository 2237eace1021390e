// Block-dense sparse attention on gfx950 MFMA: every causal key tile is
// streamed once per 128-row query block and the exact top-k selection is
// applied as a bitmask, so masked-out keys get probability 0.  Same function
// as the gather kernel (softmax over each row's selected keys), different
// work: dense MFMA over the causal triangle instead of per-row gathers.
//
// Layouts: q, k [B,T,H,128]; v stored transposed, V^T [B,H,128,ldv] (written
// once by prologue_vt_kernel) so a key tile of V^T stages straight into LDS;
// selection bits [B,T,W] uint32, W = 2*ceil(Tkv/64): bit j of row t set iff
// key j is selected and valid for query t.
//
// Per block: one head, 128 query rows, 4 waves of 32 rows, 64-key tiles
// staged in LDS.  With v_mfma_f32_32x32x16_bf16 both products are computed
// transposed,
//   S^T = K Q^T    (A = K tile from LDS, B = this wave's q, in registers)
//   O^T = V^T P^T  (A = V^T tile from LDS, B = P in registers)
// so in both outputs lane l holds column l%32 = one query row: a query's
// softmax state lives in its two lanes (l and l^32) and P never moves between
// lanes.  Accumulator r of lane l is row 8*(r/4) + 4*(l/32) + r%4 of the
// 32x32 block: keys of S^T, head dims of O^T.
#include "gsa_common.h"

namespace gsa {

constexpr int kDQ = 128;         // query rows per block (32 per wave)
constexpr int kDK = 64;          // keys per tile
constexpr int kKS = 128 + 8;     // LDS row stride of the K tile (elements): conflict-free 16-B reads
constexpr int kVS = kDK + 12;    // LDS row stride of the V^T tile (elements): conflict-free 8-B reads

// ---------------------------------------------------------------------------
// Producer with transposed V: k_out = RoPE(k) [B,T,H,128], vt = (v*sigmoid(vg))^T
// [B,H,128,ldv]; keys in [T, ldv) of vt are written as zeros.  One block per
// (b, h, 64-key tile).
// ---------------------------------------------------------------------------
struct ProVtArgs {
  const uint16_t* k; int64_t k_sb, k_st;
  const uint16_t* v; int64_t v_sb, v_st;
  const uint16_t* vg; int64_t g_sb, g_st;
  const uint16_t* cos; const uint16_t* sin; int64_t cs_st;
  uint16_t* k_out;
  uint16_t* vt;
  int T, H, ldv, ntiles;
};

__global__ __launch_bounds__(256) void prologue_vt_kernel(ProVtArgs p) {
  __shared__ __align__(16) uint16_t sV[kDK * kKS];
  const int kt = blockIdx.x % p.ntiles;
  const int bh = blockIdx.x / p.ntiles;
  const int h = bh % p.H, b = bh / p.H;
  const int j0 = kt * kDK;
  const int tid = threadIdx.x, li = tid & 15;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int item = it * 256 + tid;
    const int key = item >> 4, c = item & 15;   // c == li: one key per 16-lane row
    const int j = j0 + key;
    u32x4 packed = {0u, 0u, 0u, 0u};
    if (j < p.T) {
      if (p.k) {
        float x[8], cs[8], sn[8];
        load8(p.k + b * p.k_sb + (int64_t)j * p.k_st + h * 128 + c * 8, x);
        load8(p.cos + (int64_t)j * p.cs_st + c * 8, cs);
        load8(p.sin + (int64_t)j * p.cs_st + c * 8, sn);
        rope8<uint16_t>(x, cs, sn, li);
        store8(p.k_out + (((int64_t)b * p.T + j) * p.H + h) * 128 + c * 8, x);
      }
      float vv[8], gg[8];
      load8(p.v + b * p.v_sb + (int64_t)j * p.v_st + h * 128 + c * 8, vv);
      load8(p.vg + b * p.g_sb + (int64_t)j * p.g_st + h * 128 + c * 8, gg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = round_bf16(vv[2 * i] * round_bf16(sigmoidf_fast(gg[2 * i])));
        const float z = round_bf16(vv[2 * i + 1] * round_bf16(sigmoidf_fast(gg[2 * i + 1])));
        packed[i] = pack_bf16(a, z);
      }
    }
    *reinterpret_cast<u32x4*>(sV + key * kKS + c * 8) = packed;
  }
  __syncthreads();
  uint16_t* vtb = p.vt + ((int64_t)b * p.H + h) * 128 * p.ldv;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int item = it * 256 + tid;
    const int d = item >> 3, c8 = item & 7;     // 128 rows x 8 chunks of 8 keys
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)sV[(8 * c8 + 2 * i) * kKS + d] | ((uint32_t)sV[(8 * c8 + 2 * i + 1) * kKS + d] << 16);
    *reinterpret_cast<u32x4*>(vtb + (int64_t)d * p.ldv + j0 + 8 * c8) = w;
  }
}

// ---------------------------------------------------------------------------
// Selection bitmask from (indices, count, mask): one block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void selection_mask_kernel(
    const int32_t* __restrict__ idx, int64_t i_sb, int64_t i_st, int k_sel,
    const int32_t* __restrict__ count, const uint8_t* __restrict__ mask, int T, int Tkv, int W,
    uint32_t* __restrict__ bits, int64_t b_sb, int64_t b_st) {
  extern __shared__ uint32_t sw[];
  const int row = blockIdx.x;
  const int b = row / T, t = row % T;
  for (int i = threadIdx.x; i < W; i += 256) sw[i] = 0u;
  __syncthreads();
  int n = k_sel;
  if (count) n = min(n, count[row]);
  const int64_t base = b * i_sb + (int64_t)t * i_st;
  for (int m = threadIdx.x; m < n; m += 256) {
    if (mask == nullptr || mask[base + m] != 0) {
      const int j = min(max(idx[base + m], 0), Tkv - 1);
      atomicOr(&sw[j >> 5], 1u << (j & 31));
    }
  }
  __syncthreads();
  uint32_t* brow = bits + b * b_sb + (int64_t)t * b_st;
  for (int i = threadIdx.x; i < W; i += 256) brow[i] = sw[i];
}

// ---------------------------------------------------------------------------
// Selection bitmask -> per-lane masks of the dense kernel's score slots.
// For 32-row group g (rows 32g + i), 64-key tile kt and score slot
// s = 16c + r (c = 0,1; r = 0..15), lm[b][g][kt][s] bit (32h + i) is the
// selection bit of row 32g+i and key 64kt + 32c + 8*(r/4) + 4h + r%4 -- the
// key that accumulator r of lane (h, i) holds in the S^T MFMA output.  One
// wave per (b, g, kt).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void lane_mask_kernel(const uint32_t* __restrict__ bits, int64_t b_sb,
                                                        int64_t b_st, int T, int G, int NT, int nwaves,
                                                        uint64_t* __restrict__ lm) {
  const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= nwaves) return;
  const int kt = wv % NT, bg = wv / NT;
  const int g = bg % G, b = bg / G;
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
  const int row = 32 * g + i;
  uint64_t word = row < T ? *reinterpret_cast<const uint64_t*>(bits + b * b_sb + (int64_t)row * b_st + 2 * kt) : 0ull;
  word >>= 4 * h;
  // lane s collects slot s's mask; lanes 0..31 then write 256 contiguous bytes
  uint64_t mine = 0ull;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint64_t m = ballot64((word >> (32 * c + 8 * (r >> 2) + (r & 3))) & 1ull);
      mine = lane == 16 * c + r ? m : mine;
    }
  if (lane < 32) lm[((int64_t)bg * NT + kt) * 32 + lane] = mine;
}

// ---------------------------------------------------------------------------
// Dense masked attention (bf16)
// ---------------------------------------------------------------------------
struct DenseArgs {
  const uint16_t* q; int64_t q_sb, q_st;
  const uint16_t* k; int64_t k_sb, k_st;
  const uint16_t* vt; int64_t vt_sb, vt_sh; int ldv;
  const uint64_t* lm; int G, NT;          // lane masks [B][G][NT][32]
  const uint16_t* og; int64_t o_sb, o_st;
  const uint16_t* cos; const uint16_t* sin; int64_t cs_st;
  uint16_t* out; int64_t out_sb, out_st;
  int B, T, Tkv, H, nqb;
  float scale_l2;
  int flags;
};

constexpr int kDenseCausal = 1 << 8;   // internal flag: skip key tiles after the block's last row
constexpr float kLazy = 8.f;           // log2 headroom of the lazy softmax reference

typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Two fp32 -> packed bf16 (round to nearest even, hardware convert).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__global__ __launch_bounds__(256, 2) void dense_attn_kernel(DenseArgs p) {
  __shared__ __align__(16) uint16_t sK[kDK * kKS];
  __shared__ __align__(16) uint16_t sVt[128 * kVS];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i32 = lane & 31, h = lane >> 5;
  // heaviest query blocks first
  const int nbh = p.B * p.H;
  const int qb = p.nqb - 1 - (int)(blockIdx.x / nbh);
  const int rem = blockIdx.x % nbh;
  const int b = rem / p.H, hd = rem % p.H;
  const int q0 = qb * kDQ;
  const int qrow = q0 + 32 * w + i32;
  const int qr = min(qrow, p.T - 1);

  // ---- q: B operand of S^T; lane supplies d = 16s + 8h .. +7 of its row ----
  u32x4 qraw[8];
  const uint16_t* qp = p.q + b * p.q_sb + (int64_t)qr * p.q_st + hd * 128;
#pragma unroll
  for (int s = 0; s < 8; ++s) qraw[s] = *reinterpret_cast<const u32x4*>(qp + 16 * s + 8 * h);
  if (p.flags & GSA_ATTN_ROPE_Q) {
    // rotate_half partner of d (d < 64: -x[d+64]; else x[d-64]) is register s^4
    float x[8][8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) { x[s][2 * j] = bf16lo(qraw[s][j]); x[s][2 * j + 1] = bf16hi(qraw[s][j]); }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      float c[8], sn[8], y[8];
      load8(p.cos + (int64_t)qr * p.cs_st + 16 * s + 8 * h, c);
      load8(p.sin + (int64_t)qr * p.cs_st + 16 * s + 8 * h, sn);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = round_bf16(x[s][j] * c[j]);
        const float r = round_bf16((s < 4 ? -x[s + 4][j] : x[s - 4][j]) * sn[j]);
        y[j] = round_bf16(a + r);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) qraw[s][j] = pack_bf16(y[2 * j], y[2 * j + 1]);
    }
  }
  bf16x8 qop[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) qop[s] = __builtin_bit_cast(bf16x8, qraw[s]);

  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m = -__builtin_inff(), l = 0.f;

  const int last_key = (p.flags & kDenseCausal) ? min(p.Tkv - 1, q0 + kDQ - 1) : p.Tkv - 1;
  const int nkt = last_key / kDK + 1;
  const uint16_t* kbase = p.k + b * p.k_sb + hd * 128;
  const uint16_t* vtb = p.vt + b * p.vt_sb + hd * p.vt_sh;
  // this wave's lane masks: group 4*qb + w (wave index made uniform for scalar loads)
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const uint64_t* lmw = p.lm + ((int64_t)b * p.G + 4 * qb + wu) * p.NT * 32;

  // staging: K tile = 64 keys x 16 chunks of 16 B, V^T tile = 128 rows x 8 chunks
  u32x4 kreg[4], vreg[4];
  auto fetch = [&](int kt) {
    const int j0 = kt * kDK;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int item = it * 256 + tid;
      const int key = item >> 4, c = item & 15;
      const int j = j0 + key;
      kreg[it] = j < p.Tkv ? *reinterpret_cast<const u32x4*>(kbase + (int64_t)j * p.k_st + c * 8)
                           : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int item = it * 256 + tid;
      const int d = item >> 3, c8 = item & 7;
      vreg[it] = *reinterpret_cast<const u32x4*>(vtb + (int64_t)d * p.ldv + j0 + 8 * c8);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int item = it * 256 + tid;
      const int key = item >> 4, c = item & 15;
      *reinterpret_cast<u32x4*>(sK + key * kKS + c * 8) = kreg[it];
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int item = it * 256 + tid;
      const int d = item >> 3, c8 = item & 7;
      uint2* dst = reinterpret_cast<uint2*>(sVt + d * kVS + 8 * c8);
      dst[0] = uint2{vreg[it][0], vreg[it][1]};
      dst[1] = uint2{vreg[it][2], vreg[it][3]};
    }
  };

  fetch(0);
  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();   // the previous tile's LDS reads are done
    stash();
    __syncthreads();
    if (kt + 1 < nkt) fetch(kt + 1);   // next tile's loads fly during this tile's math

    const uint64_t* lmt = lmw + kt * 32;   // 32 slot masks of this tile

    // ---- S^T = K Q^T: two 32-key subtiles ----
    floatx16 sacc[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      floatx16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const bf16x8 ka = *reinterpret_cast<const bf16x8*>(sK + (32 * c + i32) * kKS + 16 * s + 8 * h);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qop[s], acc, 0, 0, 0);
      }
      sacc[c] = acc;
    }

    // ---- masked online softmax (log2 domain, lazy reference max) ----
    // p = 2^(s*scale*log2e - m) against a per-row reference m that only moves
    // when the row max exceeds it by more than kLazy: p <= 2^kLazy, so O and l
    // are rescaled rarely; out = O / l does not depend on m.
    float mx = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool sel = __builtin_amdgcn_inverse_ballot_w64(lmt[16 * c + r]);
        sacc[c][r] = sel ? sacc[c][r] : -__builtin_inff();
        mx = fmaxf(mx, sacc[c][r]);
      }
    mx = fmaxf(mx, xor32(mx)) * p.scale_l2;
    const bool bump = mx > m + kLazy || (m == -__builtin_inff() && mx != -__builtin_inff());
    const float mref = bump ? mx : m;
    const float alpha = bump ? __builtin_amdgcn_exp2f(m - mx) : 1.f;   // m = -inf -> 0
    const float msafe = mref == -__builtin_inff() ? 0.f : mref;
    // P as the B operand of O^T: k-step ks = 2c + s2 covers keys
    // 32c + 16*s2 + 4h + {0..3} and 32c + 16*s2 + 8 + 4h + {0..3}
    uint32_t pk[4][4];
    float lsum = 0.f;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[c][r], p.scale_l2, -msafe));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[c][r + 1], p.scale_l2, -msafe));
        pk[2 * c + (r >> 3)][(r & 7) >> 1] = cvt_pk_bf16(p0, p1);
        lsum += p0 + p1;
      }
    l = l * alpha + lsum;
    if (ballot64(bump)) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
    }
    m = mref;

    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{pk[ks][0], pk[ks][1], pk[ks][2], pk[ks][3]});
      const int koff = 32 * (ks >> 1) + 16 * (ks & 1) + 4 * h;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t* vr = sVt + (32 * dt + i32) * kVS + koff;
        const uint2 a0 = *reinterpret_cast<const uint2*>(vr);
        const uint2 a1 = *reinterpret_cast<const uint2*>(vr + 8);
        const bf16x8 va = __builtin_bit_cast(bf16x8, u32x4{a0.x, a0.y, a1.x, a1.y});
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, o[dt], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: normalise, bf16, optional output gate ----
  l += xor32(l);
  if (qrow < p.T) {
    uint16_t* op = p.out + b * p.out_sb + (int64_t)qrow * p.out_st + hd * 128;
    const uint16_t* gp = (p.flags & GSA_ATTN_OUT_GATE) ? p.og + b * p.o_sb + (int64_t)qrow * p.o_st + hd * 128
                                                       : nullptr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * dt + 8 * r4 + 4 * h;
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = round_bf16(l > 0.f ? o[dt][4 * r4 + e] / l : 0.f);
        if (gp) {
          const uint2 gw = *reinterpret_cast<const uint2*>(gp + d0);
          const float gl[4] = {bf16lo(gw.x), bf16hi(gw.x), bf16lo(gw.y), bf16hi(gw.y)};
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = round_bf16(r[e] * round_bf16(sigmoidf_fast(gl[e])));
        }
        *reinterpret_cast<uint2*>(op + d0) = uint2{pack_bf16(r[0], r[1]), pack_bf16(r[2], r[3])};
      }
  }
}

}  // namespace gsa

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
using namespace gsa_host;

extern "C" int gsa_prologue_vt(const void* k, int64_t k_sb, int64_t k_st,
                               const void* v, int64_t v_sb, int64_t v_st,
                               const void* vg, int64_t g_sb, int64_t g_st,
                               const void* cos, const void* sin, int64_t cs_st,
                               int B, int T, int H, int d, int dtype,
                               void* k_out, void* vt, int ldv,
                               void* stream) {
  if (!v || !vg || !vt) return GSA_ERR_NULL;
  if (k && (!cos || !sin || !k_out)) return GSA_ERR_NULL;
  if (dtype != GSA_DTYPE_BF16) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || d != 128 || H < 1 || H > 64) return GSA_ERR_SHAPE;
  if (ldv < T || ldv % 64 != 0) return GSA_ERR_SHAPE;
  if ((int64_t)B * H * (ldv / 64) > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!vec_ok(v, v_sb, v_st, dtype) || !vec_ok(vg, g_sb, g_st, dtype) || !aligned(vt, 16)) return GSA_ERR_ALIGN;
  if (k && (!vec_ok(k, k_sb, k_st, dtype) || !vec_ok(cos, 0, cs_st, dtype) || !vec_ok(sin, 0, cs_st, dtype) ||
            !aligned(k_out, 16)))
    return GSA_ERR_ALIGN;
  gsa::ProVtArgs a{static_cast<const uint16_t*>(k), k_sb, k_st, static_cast<const uint16_t*>(v), v_sb, v_st,
                   static_cast<const uint16_t*>(vg), g_sb, g_st, static_cast<const uint16_t*>(cos),
                   static_cast<const uint16_t*>(sin), cs_st, static_cast<uint16_t*>(k_out),
                   static_cast<uint16_t*>(vt), T, H, ldv, ldv / 64};
  hipLaunchKernelGGL(gsa::prologue_vt_kernel, dim3(B * H * (ldv / 64)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}

extern "C" int gsa_selection_mask(const int32_t* idx, int64_t i_sb, int64_t i_st, int k_sel,
                                  const int32_t* count, const uint8_t* mask,
                                  int B, int T, int Tkv, uint32_t* bits, int64_t b_sb, int64_t b_st,
                                  void* stream) {
  if (!idx || !bits) return GSA_ERR_NULL;
  if (B < 1 || T < 1 || Tkv < 1 || k_sel < 0) return GSA_ERR_SHAPE;
  const int W = 2 * ((Tkv + 63) / 64);
  if ((size_t)W * 4 > 65536) return GSA_ERR_SHAPE;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!aligned(idx, 4) || !aligned(bits, 8) || (b_st % 2) || (b_sb % 2) || (count && !aligned(count, 4)))
    return GSA_ERR_ALIGN;
  hipLaunchKernelGGL(gsa::selection_mask_kernel, dim3(B * T), dim3(256), (size_t)W * 4,
                     static_cast<hipStream_t>(stream), idx, i_sb, i_st, k_sel, count, mask, T, Tkv, W, bits,
                     b_sb, b_st);
  return launch_status();
}

extern "C" size_t gsa_dense_attn_workspace_bytes(int B, int T, int Tkv) {
  if (B < 1 || T < 1 || Tkv < 1) return 0;
  return (size_t)B * ((T + 31) / 32) * ((Tkv + 63) / 64) * 32 * sizeof(uint64_t);
}

extern "C" int gsa_dense_attn(const void* q, int64_t q_sb, int64_t q_st,
                              const void* k, int64_t k_sb, int64_t k_st,
                              const void* vt, int64_t vt_sb, int64_t vt_sh, int ldv,
                              const uint32_t* bits, int64_t b_sb, int64_t b_st,
                              const void* og, int64_t o_sb, int64_t o_st,
                              const void* cos, const void* sin, int64_t cs_st,
                              void* out, int64_t out_sb, int64_t out_st,
                              int B, int T, int Tkv, int H, int d, float scale,
                              int dtype, int flags, int causal,
                              void* ws, size_t ws_bytes,
                              void* stream) {
  if (!q || !k || !vt || !bits || !out || !ws) return GSA_ERR_NULL;
  if (flags & ~(GSA_ATTN_ROPE_Q | GSA_ATTN_OUT_GATE)) return GSA_ERR_FLAGS;
  if ((flags & GSA_ATTN_ROPE_Q) && (!cos || !sin)) return GSA_ERR_NULL;
  if ((flags & GSA_ATTN_OUT_GATE) && !og) return GSA_ERR_NULL;
  if (dtype != GSA_DTYPE_BF16) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || Tkv < 1 || d != 128 || H < 1 || H > 64) return GSA_ERR_SHAPE;
  const int NT = (Tkv + 63) / 64;
  if (ldv < NT * 64 || ldv % 64 != 0) return GSA_ERR_SHAPE;
  if (b_st < 2 * NT || (B > 1 && b_sb < (int64_t)T * b_st)) return GSA_ERR_SHAPE;
  if (ws_bytes < gsa_dense_attn_workspace_bytes(B, T, Tkv)) return GSA_ERR_SHAPE;
  const int nqb = (T + gsa::kDQ - 1) / gsa::kDQ;
  const int G = nqb * (gsa::kDQ / 32);    // 32-row groups, padded to whole blocks
  if ((int64_t)B * H * nqb > 0x7fffffffLL || (int64_t)B * G * NT > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!vec_ok(q, q_sb, q_st, dtype) || !vec_ok(k, k_sb, k_st, dtype) || !vec_ok(vt, vt_sb, vt_sh, dtype) ||
      !vec_ok(out, out_sb, out_st, dtype) || !aligned(bits, 8) || (b_sb % 2) || (b_st % 2) || !aligned(ws, 8))
    return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_OUT_GATE) && !vec_ok(og, o_sb, o_st, dtype)) return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_ROPE_Q) && (!vec_ok(cos, 0, cs_st, dtype) || !vec_ok(sin, 0, cs_st, dtype)))
    return GSA_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint64_t* lm = static_cast<uint64_t*>(ws);
  const int nwaves = B * G * NT;
  hipLaunchKernelGGL(gsa::lane_mask_kernel, dim3((nwaves + 3) / 4), dim3(256), 0, s, bits, b_sb, b_st, T, G, NT,
                     nwaves, lm);
  int st = launch_status();
  if (st) return st;
  gsa::DenseArgs a{static_cast<const uint16_t*>(q), q_sb, q_st, static_cast<const uint16_t*>(k), k_sb, k_st,
                   static_cast<const uint16_t*>(vt), vt_sb, vt_sh, ldv, lm, G, NT,
                   static_cast<const uint16_t*>(og), o_sb, o_st, static_cast<const uint16_t*>(cos),
                   static_cast<const uint16_t*>(sin), cs_st, static_cast<uint16_t*>(out), out_sb, out_st,
                   B, T, Tkv, H, nqb, scale * gsa::kLog2e, flags | (causal ? gsa::kDenseCausal : 0)};
  hipLaunchKernelGGL(gsa::dense_attn_kernel, dim3(B * H * nqb), dim3(256), 0, s, a);
  return launch_status();
}
