// Sparse gather-attention and its producer pass, gfx950.
//
// Thread mapping (both kernels): one block per query row (b, t) with 16 lanes
// per head -- a 16-lane DPP row -- and each lane owning 8 consecutive
// elements of its head's 128.  A key row of all H heads (H*256 bytes in bf16)
// is therefore one 16-byte load per lane, contiguous across the block, and a
// head's dot product is 8 MACs per lane plus a 4-step DPP reduction.
//
// Rounding: in bf16 every elementwise op the reference performs in bf16
// (RoPE's two products and sum, the gate sigmoids and products, the cast of
// the attention output) is rounded to bf16 at the same point, so those values
// match the reference's bf16 results; everything else accumulates in fp32.
#include "gsa_common.h"

// Products and sums round one at a time, as torch rounds them.
#pragma clang fp contract(off)

namespace gsa {

// ---------------------------------------------------------------------------
// Producer: k_out = RoPE(k) and/or v_out = v * sigmoid(vg)  (block = 16*H threads)
// ---------------------------------------------------------------------------
struct ProArgs {
  const void* k; int64_t k_sb, k_st;
  const void* v; int64_t v_sb, v_st;
  const void* vg; int64_t g_sb, g_st;
  const void* cos; const void* sin; int64_t cs_st;
  void* k_out; void* v_out;
  int T, HD;   // HD = H * 128
};

template <typename T>
__global__ __launch_bounds__(1024) void prologue_kernel(ProArgs p) {
  const int row = blockIdx.x;
  const int b = row / p.T, t = row % p.T;
  const int li = threadIdx.x & 15;
  const int e0 = threadIdx.x * 8;   // == head*128 + li*8
  const int64_t o = (int64_t)row * p.HD + e0;
  if (p.k) {
    float x[8], c[8], s[8];
    load8(static_cast<const T*>(p.k) + b * p.k_sb + (int64_t)t * p.k_st + e0, x);
    load8(static_cast<const T*>(p.cos) + (int64_t)t * p.cs_st + li * 8, c);
    load8(static_cast<const T*>(p.sin) + (int64_t)t * p.cs_st + li * 8, s);
    rope8<T>(x, c, s, li);
    store8(static_cast<T*>(p.k_out) + o, x);
  }
  if (p.v) {
    float vv[8], gg[8];
    load8(static_cast<const T*>(p.v) + b * p.v_sb + (int64_t)t * p.v_st + e0, vv);
    load8(static_cast<const T*>(p.vg) + b * p.g_sb + (int64_t)t * p.g_st + e0, gg);
#pragma unroll
    for (int i = 0; i < 8; ++i) vv[i] = Elem<T>::rnd(vv[i] * Elem<T>::rnd(sigmoidf_fast(gg[i])));
    store8(static_cast<T*>(p.v_out) + o, vv);
  }
}

// ---------------------------------------------------------------------------
// Sparse attention
// ---------------------------------------------------------------------------
struct AttnArgs {
  const void* q; int64_t q_sb, q_st;
  const void* k; int64_t k_sb, k_st;
  const void* v; int64_t v_sb, v_st;
  const int32_t* idx; int64_t i_sb, i_st; int k_sel;
  const int32_t* count; const uint8_t* mask;
  const void* og; int64_t o_sb, o_st;
  const void* cos; const void* sin; int64_t cs_st;
  void* out; int64_t out_sb, out_st;
  int T, Tkv;
  float scale_l2;   // scale * log2(e): scores live in the log2 domain
  int flags;
};

// One key row slice for this lane: 8 elements as raw storage.
template <typename T> struct KV;
template <> struct KV<uint16_t> {
  u32x4 r;
  __device__ void load(const uint16_t* p) { r = *reinterpret_cast<const u32x4*>(p); }
  __device__ float dot(const float (&q)[8]) const {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = __builtin_fmaf(q[2 * i], bf16lo(r[i]), acc);
      acc = __builtin_fmaf(q[2 * i + 1], bf16hi(r[i]), acc);
    }
    return acc;
  }
  __device__ void axpy(float p, float (&acc)[8]) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = __builtin_fmaf(p, bf16lo(r[i]), acc[2 * i]);
      acc[2 * i + 1] = __builtin_fmaf(p, bf16hi(r[i]), acc[2 * i + 1]);
    }
  }
};
template <> struct KV<float> {
  floatx4 a, b;
  __device__ void load(const float* p) {
    a = *reinterpret_cast<const floatx4*>(p);
    b = *reinterpret_cast<const floatx4*>(p + 4);
  }
  __device__ float dot(const float (&q)[8]) const {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(q[i], a[i], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(q[4 + i], b[i], acc);
    return acc;
  }
  __device__ void axpy(float p, float (&acc)[8]) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(p, a[i], acc[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[4 + i] = __builtin_fmaf(p, b[i], acc[4 + i]);
  }
};

// q held as fp32 (exact for bf16 inputs).
struct QReg {
  float r[8];
  __device__ void set(const float (&x)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = x[i];
  }
  __device__ const float (&op() const)[8] { return r; }
};

template <typename T> struct Chunk { static constexpr int kKeys = 8; };
template <> struct Chunk<float> { static constexpr int kKeys = 4; };

template <typename T, int kThreads>
__global__ __launch_bounds__(kThreads) void sparse_attn_kernel(AttnArgs p) {
  // keys in flight per buffer; halved for 1024-thread blocks (128-VGPR budget)
  constexpr int C = kThreads > 256 ? Chunk<T>::kKeys / 2 : Chunk<T>::kKeys;
  const int row = blockIdx.x;
  const int b = row / p.T, t = row % p.T;
  const int li = threadIdx.x & 15;
  const int e0 = threadIdx.x * 8;   // head*128 + li*8

  // ---- q (optionally RoPE'd here) ----
  float xq[8];
  load8(static_cast<const T*>(p.q) + b * p.q_sb + (int64_t)t * p.q_st + e0, xq);
  if (p.flags & GSA_ATTN_ROPE_Q) {
    float c[8], s[8];
    load8(static_cast<const T*>(p.cos) + (int64_t)t * p.cs_st + li * 8, c);
    load8(static_cast<const T*>(p.sin) + (int64_t)t * p.cs_st + li * 8, s);
    rope8<T>(xq, c, s, li);
  }
  QReg q;
  q.set(xq);

  const int32_t* irow = p.idx + b * p.i_sb + (int64_t)t * p.i_st;
  const uint8_t* mrow = p.mask ? p.mask + b * p.i_sb + (int64_t)t * p.i_st : nullptr;
  int n = p.k_sel;
  if (p.count) n = min(n, p.count[row]);
  const T* kb = static_cast<const T*>(p.k) + b * p.k_sb + e0;
  const T* vb = static_cast<const T*>(p.v) + b * p.v_sb + e0;

  float m = -__builtin_inff(), l = 0.f;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;

  KV<T> kc[C], vc[C], kn[C], vn[C];
  bool okc[C], okn[C];

  auto fetch = [&](int c0, KV<T> (&kr)[C], KV<T> (&vr)[C], bool (&ok)[C]) {
#pragma unroll
    for (int u = 0; u < C; ++u) {
      const int mm = c0 + u;
      ok[u] = mm < n && (mrow == nullptr || mrow[mm] != 0);
      if (ok[u]) {
        const int j = min(max(irow[mm], 0), p.Tkv - 1);
        kr[u].load(kb + (int64_t)j * p.k_st);
        vr[u].load(vb + (int64_t)j * p.v_st);
      }
    }
  };

  auto consume = [&](const KV<T> (&kr)[C], const KV<T> (&vr)[C], const bool (&ok)[C]) {
    float s[C];
    float mx = m;
#pragma unroll
    for (int u = 0; u < C; ++u) {
      s[u] = ok[u] ? row16_sum(kr[u].dot(q.op())) * p.scale_l2 : -__builtin_inff();
      mx = fmaxf(mx, s[u]);
    }
    if (mx == -__builtin_inff()) return;   // nothing valid yet (uniform per row)
    const float alpha = __builtin_amdgcn_exp2f(m - mx);   // m = -inf -> 0
    l *= alpha;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
    for (int u = 0; u < C; ++u) {
      if (ok[u]) {
        const float pu = __builtin_amdgcn_exp2f(s[u] - mx);
        l += pu;
        vr[u].axpy(pu, acc);
      }
    }
    m = mx;
  };

  if (n > 0) {
    fetch(0, kc, vc, okc);
    for (int c0 = 0; c0 < n; c0 += 2 * C) {
      if (c0 + C < n) fetch(c0 + C, kn, vn, okn);
      consume(kc, vc, okc);
      if (c0 + C >= n) break;
      if (c0 + 2 * C < n) fetch(c0 + 2 * C, kc, vc, okc);
      consume(kn, vn, okn);
    }
  }

  // ---- epilogue: normalise, cast, optional output gate ----
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = Elem<T>::rnd(l > 0.f ? acc[i] / l : 0.f);
  if (p.flags & GSA_ATTN_OUT_GATE) {
    float gg[8];
    load8(static_cast<const T*>(p.og) + b * p.o_sb + (int64_t)t * p.o_st + e0, gg);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = Elem<T>::rnd(o[i] * Elem<T>::rnd(sigmoidf_fast(gg[i])));
  }
  store8(static_cast<T*>(p.out) + b * p.out_sb + (int64_t)t * p.out_st + e0, o);
}

}  // namespace gsa

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
using namespace gsa_host;

extern "C" int gsa_prologue(const void* k, int64_t k_sb, int64_t k_st,
                            const void* v, int64_t v_sb, int64_t v_st,
                            const void* vg, int64_t g_sb, int64_t g_st,
                            const void* cos, const void* sin, int64_t cs_st,
                            int B, int T, int H, int d, int dtype,
                            void* k_out, void* v_out,
                            void* stream) {
  const bool do_k = k != nullptr, do_v = v != nullptr;
  if (!do_k && !do_v) return GSA_ERR_NULL;
  if (do_k && (!cos || !sin || !k_out)) return GSA_ERR_NULL;
  if (do_v && (!vg || !v_out)) return GSA_ERR_NULL;
  if (dtype_size(dtype) == 0) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || d != 128 || H < 1 || H > 64) return GSA_ERR_SHAPE;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (do_k && (!vec_ok(k, k_sb, k_st, dtype) || !vec_ok(cos, 0, cs_st, dtype) ||
               !vec_ok(sin, 0, cs_st, dtype) || !aligned(k_out, 16)))
    return GSA_ERR_ALIGN;
  if (do_v && (!vec_ok(v, v_sb, v_st, dtype) || !vec_ok(vg, g_sb, g_st, dtype) || !aligned(v_out, 16)))
    return GSA_ERR_ALIGN;
  gsa::ProArgs a{k, k_sb, k_st, v, v_sb, v_st, vg, g_sb, g_st, cos, sin, cs_st, k_out, v_out, T, H * 128};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GSA_DTYPE_BF16)
    hipLaunchKernelGGL(gsa::prologue_kernel<uint16_t>, dim3(B * T), dim3(16 * H), 0, s, a);
  else
    hipLaunchKernelGGL(gsa::prologue_kernel<float>, dim3(B * T), dim3(16 * H), 0, s, a);
  return launch_status();
}

extern "C" int gsa_sparse_attn(const void* q, int64_t q_sb, int64_t q_st,
                               const void* k, int64_t k_sb, int64_t k_st,
                               const void* v, int64_t v_sb, int64_t v_st,
                               const int32_t* idx, int64_t i_sb, int64_t i_st, int k_sel,
                               const int32_t* count, const uint8_t* mask,
                               const void* og, int64_t o_sb, int64_t o_st,
                               const void* cos, const void* sin, int64_t cs_st,
                               void* out, int64_t out_sb, int64_t out_st,
                               int B, int T, int Tkv, int H, int d, float scale,
                               int dtype, int flags,
                               void* stream) {
  if (!q || !k || !v || !idx || !out) return GSA_ERR_NULL;
  if (flags & ~(GSA_ATTN_ROPE_Q | GSA_ATTN_OUT_GATE)) return GSA_ERR_FLAGS;
  if ((flags & GSA_ATTN_ROPE_Q) && (!cos || !sin)) return GSA_ERR_NULL;
  if ((flags & GSA_ATTN_OUT_GATE) && !og) return GSA_ERR_NULL;
  if (dtype_size(dtype) == 0) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || Tkv < 1 || d != 128 || H < 1 || H > 64) return GSA_ERR_SHAPE;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (k_sel < 0) return GSA_ERR_K;
  if (!vec_ok(q, q_sb, q_st, dtype) || !vec_ok(k, k_sb, k_st, dtype) || !vec_ok(v, v_sb, v_st, dtype) ||
      !vec_ok(out, out_sb, out_st, dtype) || !aligned(idx, 4) || (count && !aligned(count, 4)))
    return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_OUT_GATE) && !vec_ok(og, o_sb, o_st, dtype)) return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_ROPE_Q) && (!vec_ok(cos, 0, cs_st, dtype) || !vec_ok(sin, 0, cs_st, dtype)))
    return GSA_ERR_ALIGN;
  gsa::AttnArgs a{q, q_sb, q_st, k, k_sb, k_st, v, v_sb, v_st, idx, i_sb, i_st, k_sel, count, mask,
                  og, o_sb, o_st, cos, sin, cs_st, out, out_sb, out_st, T, Tkv,
                  scale * gsa::kLog2e, flags};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(B * T), block(16 * H);
  if (dtype == GSA_DTYPE_BF16) {
    if (H <= 16) hipLaunchKernelGGL((gsa::sparse_attn_kernel<uint16_t, 256>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gsa::sparse_attn_kernel<uint16_t, 1024>), grid, block, 0, s, a);
  } else {
    if (H <= 16) hipLaunchKernelGGL((gsa::sparse_attn_kernel<float, 256>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((gsa::sparse_attn_kernel<float, 1024>), grid, block, 0, s, a);
  }
  return launch_status();
}
