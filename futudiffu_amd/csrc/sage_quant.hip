// Memory-bound front half of the Sage forward on gfx950: K smoothing and
// Q/K/V quantization into MFMA-fragment order.
//
// Reference semantics (sqcu/futudiffu):
//   smoothing        src/futudiffu/sage_attention.py:63-71 (k - k.mean(dim=2))
//   Q int8 / fp8     src/futudiffu/sage_kernels.py:1415-1422 / :250-258
//   K int8 / fp8     src/futudiffu/sage_kernels.py:1443-1449 / :272-280
//   V fp8            src/futudiffu/sage_kernels.py:1143-1148
// The reference re-quantizes K for every 128-row Q tile inside the attention
// loop; per-token scales depend only on the token, so quantizing once here
// yields identical codes.
//
// With smoothing, k_colsum first reads K once and writes fp64 column sums of
// each 256-token chunk (no atomics, nothing to clear beforehand).  quantize
// (one workgroup per 64-token block and head) then issues all of its Q, K and
// V loads up front, adds the chunk sums of its head in a fixed order to form
// the mean, and writes the Q, K and V codes.  The mean makes the second read
// of K unavoidable: every K code depends on all N tokens.
#include "sage_common.h"
#include "sage_launch.h"

namespace sage {

// 8 bf16 (one 16-byte load) -> fp32.
__device__ __forceinline__ void unpack8(uint4 w, float x[8]) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = __uint_as_float(ww[e] << 16);
    x[2 * e + 1] = __uint_as_float(ww[e] & 0xffff0000u);
  }
}

// Max over aligned groups of G lanes (G in {8, 16}) with DPP row permutes:
// quad xor 1, quad xor 2, half-row mirror (8 lanes), row mirror (16 lanes).
template <int G>
__device__ __forceinline__ float group_max(float a) {
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0xB1, 0xf, 0xf, false)));  // [1,0,3,2]
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x4E, 0xf, 0xf, false)));  // [2,3,0,1]
  a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x141, 0xf, 0xf, false)));  // half mirror
  if constexpr (G == 16) a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x140, 0xf, 0xf, false)));
  return a;
}

// Max across the 16-lane rows of a wave (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float rows_max(float a) {
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
  a = fmaxf(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
  return fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t word_of(uint4 w, int i) {
  return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
}

// Quantize the 8 channels a lane holds for each of its PASSES tokens of one
// operand (Q or K) and store codes in row-fragment order plus scales.
// x holds the (smoothed) values; amax is per token, or per 64-token block.
template <int D, int QK, int GRAN, int PASSES>
__device__ __forceinline__ void store_rows(const float (&x)[PASSES][8], const float (&amax)[PASSES], int64_t tok0,
                                           int rr, int c8, float fold, uint8_t* __restrict__ codes,
                                           float* __restrict__ scale, int tid) {
  constexpr int RPP = 256 / (D / 8);
  const float qmax = (QK == kQK_INT8) ? kInt8Max : kFp8Max;
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t tok = tok0 + rr + ps * RPP;
    const float inv = qmax / fmaxf(amax[ps], kEps);  // IEEE division (correctly rounded)
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = x[ps][e] * inv;
    uint2 word;
    if (QK == kQK_INT8) {
      word.x = pack_i8x4(y[0], y[1], y[2], y[3]);
      word.y = pack_i8x4(y[4], y[5], y[6], y[7]);
    } else {
      word.x = pack_fp8x4(y[0], y[1], y[2], y[3]);
      word.y = pack_fp8x4(y[4], y[5], y[6], y[7]);
    }
    const int d0 = c8 * 8;
    *reinterpret_cast<uint2*>(codes + row_frag_offset(tok, d0 / 32, (d0 / 16) & 1, D) + (d0 & 8)) = word;
    if (GRAN == kGRAN_TOKEN) {
      if (c8 == 0) scale[tok] = (amax[ps] / qmax) * fold;
    } else if (tid == 0 && ps == 0) {
      scale[tok0 / 64] = (amax[ps] / qmax) * fold;
    }
  }
}

// Per-token (or per-block) |x| maxima of a lane's tokens.
template <int D, int GRAN, int PASSES>
__device__ __forceinline__ void row_amax(const float (&x)[PASSES][8], float (&amax)[PASSES], unsigned int* blk_u) {
  constexpr int LPR = D / 8;
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(x[ps][e]));
    amax[ps] = group_max<LPR>(a);
  }
  if (GRAN == kGRAN_BLOCK64) {
    float a = 0.0f;
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) a = fmaxf(a, amax[ps]);
    if ((threadIdx.x % LPR) == 0) atomicMax(blk_u, __float_as_uint(a));
    __syncthreads();
    a = __uint_as_float(*blk_u);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) amax[ps] = a;
  }
}

// ---- q/k producer (fused_qkv_postprocess, fused_kernels.py:271-390) ---------

// Sum over the LPR consecutive lanes (8 or 16) that hold one token's channels:
// a pairwise tree over the lanes in order, with DPP moves of the two halves of
// the fp64 value (quad xor 1, quad xor 2, half-row mirror, row mirror, as in
// group_max).  At each step both lanes of a pair add the same two operands, so
// every lane of the token ends with the same value.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

template <int LPR>
__device__ __forceinline__ double token_sum(double v) {
  v += dpp_f64<0xB1>(v);   // [1,0,3,2]
  v += dpp_f64<0x4E>(v);   // [2,3,0,1]
  v += dpp_f64<0x141>(v);  // half-row mirror: quad q with quad q^1
  if constexpr (LPR == 16) v += dpp_f64<0x140>(v);  // row mirror: half-row with half-row
  return v;
}

// Two fp32 -> two bf16 (round to nearest even, v_cvt_pk_bf16_f32) in one word.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// RMSNorm + rotary embedding of the 8 channels [8*c8, +8) of one token held
// by a lane (bf16 in, bf16 out).  rrms = 1 / sqrt(mean(x^2) + eps) over the
// token's D channels (fused_kernels.py:316-320; the sum of squares in fp64, in
// a fixed order: each lane's 8 channels left to right, then a pairwise tree
// over the token's lanes; rounded once to fp32), n = x * rrms * w (:357-360), and per channel
// pair (2p, 2p+1) with fr[p] = (cos, -sin, sin) (:334-336):
// even' = cos*n_even + (-sin)*n_odd, odd' = sin*n_even + cos*n_odd (:363-366),
// every product and sum a separately rounded fp32 operation.
template <int D>
__device__ __forceinline__ uint4 rms_rope8(uint4 w, const float (&nw)[8], const f32x4 (&fr)[4], float eps) {
#pragma clang fp contract(off)  // no fused multiply-add: every product and sum rounds on its own
  float x[8];
  unpack8(w, x);
  double ss = 0.0;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = __builtin_fma((double)x[e], (double)x[e], ss);  // the square is exact
  ss = token_sum<D / 8>(ss);
  const float ms = (float)(ss / (double)D);
  const float rrms = 1.0f / sqrtf(ms + eps);  // correctly rounded sqrt and division
  float nn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) nn[e] = (x[e] * rrms) * nw[e];
  uint32_t o[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float re = fr[p][0] * nn[2 * p] + fr[p][1] * nn[2 * p + 1];
    const float ro = fr[p][2] * nn[2 * p] + fr[p][0] * nn[2 * p + 1];
    o[p] = pack_bf16x2(re, ro);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// The rotary matrices of channel pairs [4*c8, +4) of token `row` of the
// flattened (batch, token) axis: (cos, -sin, sin) of each pair, the three
// entries the reference reads (fused_kernels.py:334-336); the fourth lane is
// unused.  Three floats instead of the 16-byte matrix keep fewer registers
// live (measured 79.4 -> 72.7 us for the producer-fused quantization at
// 1x30x4416x128).
template <int D>
__device__ __forceinline__ void load_freqs(const float* freqs, int64_t row, int c8, f32x4 (&fr)[4]) {
  const float* fp = freqs + (row * (D / 2) + 4 * c8) * 4;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const f32x2 cs = *reinterpret_cast<const f32x2*>(fp + 4 * p);
    fr[p] = f32x4{cs[0], cs[1], fp[4 * p + 2], 0.0f};
  }
}

__device__ __forceinline__ void load_w8(const float* w, int c8, float (&out)[8]) {
  const f32x4* p = reinterpret_cast<const f32x4*>(w + 8 * c8);
  const f32x4 a = p[0], b = p[1];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[i] = a[i];
    out[4 + i] = b[i];
  }
}

// Block coordinates (unit, bh).  Reading bf16 q, k, v [BH, N, D], the 2D grid
// (units, BH) walks one head's units.  The projection output [B, N, 3*H*D]
// holds every head in each token row, so producer launches use a 1D grid with
// the head fastest: consecutive workgroups read all heads of the same rows.
template <bool PROD>
__device__ __forceinline__ void block_coords(const ProdArgs& prod, int64_t& unit, int& bh) {
  if constexpr (PROD) {
    const int64_t b = blockIdx.x;
    unit = b / prod.bh;
    bh = (int)(b - unit * prod.bh);
  } else {
    unit = blockIdx.x;
    bh = (int)blockIdx.y;
  }
}

// Source rows of one head for the quantization: bf16 q, k, v [BH, N, D], or
// (PROD) the q, k and v column blocks of head bh % h in the projection output
// [B, N, 3*h*D], whose tokens are 3*h*D elements apart.
template <int D, bool PROD>
struct HeadRows {
  const uint16_t *q, *k, *v;
  int64_t stride;  // elements between consecutive tokens
  int64_t row0;    // flattened (batch, token) index of token 0 (freqs row)
  __device__ HeadRows(const uint16_t* q_, const uint16_t* k_, const uint16_t* v_, const ProdArgs& prod, int bh,
                      int64_t n) {
    if constexpr (PROD) {
      const int b = bh / prod.h, head = bh - b * prod.h;
      stride = 3LL * prod.h * D;
      row0 = (int64_t)b * n;
      q = prod.qkv + row0 * stride + (int64_t)head * D;
      k = q + (int64_t)prod.h * D;
      v = k + (int64_t)prod.h * D;
    } else {
      stride = D;
      row0 = 0;
      q = q_ + (int64_t)bh * n * D;
      k = k_ + (int64_t)bh * n * D;
      v = v_ + (int64_t)bh * n * D;
    }
  }
};

// Standalone producer: bf16 q, k, v [BH, N, D] from the projection output
// (the outputs of fused_qkv_postprocess, fused_kernels.py:372-385).  One
// workgroup per (64-token block, bh); lane (rr, c8) holds channels
// [8*c8, +8) of tokens rr + RPP*ps.
template <int D>
__global__ void __launch_bounds__(256) qkv_postprocess_kernel(ProdArgs prod, int64_t n, uint16_t* __restrict__ q_out,
                                                              uint16_t* __restrict__ k_out,
                                                              uint16_t* __restrict__ v_out) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  int64_t unit;
  int bh;
  block_coords<true>(prod, unit, bh);
  const int tid = threadIdx.x;
  const int c8 = tid % LPR, rr = tid / LPR;
  const int64_t tok0 = unit * 64;
  const HeadRows<D, true> src(nullptr, nullptr, nullptr, prod, bh, n);
  float qn[8], kn[8];
  load_w8(prod.qw, c8, qn);
  load_w8(prod.kw, c8, kn);
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t t = tok0 + rr + ps * RPP;
    const int64_t tok = min(t, n - 1);  // clamped: the lanes of a token reduce together
    const uint4 qw = *reinterpret_cast<const uint4*>(src.q + tok * src.stride + c8 * 8);
    const uint4 kw = *reinterpret_cast<const uint4*>(src.k + tok * src.stride + c8 * 8);
    const uint4 vw = *reinterpret_cast<const uint4*>(src.v + tok * src.stride + c8 * 8);
    f32x4 fr[4];
    load_freqs<D>(prod.freqs, src.row0 + tok, c8, fr);
    const uint4 qo = rms_rope8<D>(qw, qn, fr, prod.eps);
    const uint4 ko = rms_rope8<D>(kw, kn, fr, prod.eps);
    if (t < n) {
      const int64_t o = ((int64_t)bh * n + t) * D + c8 * 8;
      *reinterpret_cast<uint4*>(q_out + o) = qo;
      *reinterpret_cast<uint4*>(k_out + o) = ko;
      *reinterpret_cast<uint4*>(v_out + o) = vw;
    }
  }
}

// Gradient of the producer with respect to the projection output
// (fused_kernels.py:711-783): per head and token, g' = the rotation's
// transpose applied to the incoming gradient (:736-758), then the RMSNorm
// backward dx = rrms * (g'w - x * rrms^2 * sum(g'w * x) / D) (:760-776) for q
// and k; v's gradient passes through; all written in the [B, N, 3*H*D]
// layout (:778-783).  fp32 arithmetic with fp64 row sums (8 channels per lane,
// then the token's lanes); the norm weights and rotations get no gradient, as
// in the reference.  One workgroup per (64-token block, head), head fastest;
// lane (rr, c8) holds channels [8*c8, +8) of tokens rr + RPP*ps.
template <int D>
__global__ void __launch_bounds__(256) qkv_postprocess_bwd_kernel(ProdArgs prod, int64_t n,
                                                                  const uint16_t* __restrict__ gq,
                                                                  const uint16_t* __restrict__ gk,
                                                                  const uint16_t* __restrict__ gv,
                                                                  uint16_t* __restrict__ dqkv) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  int64_t unit;
  int bh;
  block_coords<true>(prod, unit, bh);
  const int tid = threadIdx.x;
  const int c8 = tid % LPR, rr = tid / LPR;
  const int64_t tok0 = unit * 64;
  const HeadRows<D, true> src(nullptr, nullptr, nullptr, prod, bh, n);
  const int64_t head_off = (int64_t)(bh % prod.h) * D;  // the head's column offset in each third
  const int64_t third = (int64_t)prod.h * D;
  float qn[8], kn[8];
  load_w8(prod.qw, c8, qn);
  load_w8(prod.kw, c8, kn);
  auto one = [&](uint4 xw, uint4 gw, const float (&w)[8], const f32x4 (&fr)[4]) __attribute__((always_inline)) {
    float x[8], g[8], gp[8];
    unpack8(xw, x);
    unpack8(gw, g);
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // transpose of [[cos, -sin], [sin, cos]]
      const float c = fr[p][0], sn = fr[p][2];
      gp[2 * p] = (c * g[2 * p] + sn * g[2 * p + 1]) * w[2 * p];
      gp[2 * p + 1] = (c * g[2 * p + 1] - sn * g[2 * p]) * w[2 * p + 1];
    }
    double ss = 0.0, gx = 0.0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ss = __builtin_fma((double)x[e], (double)x[e], ss);
      gx = __builtin_fma((double)gp[e], (double)x[e], gx);
    }
    ss = token_sum<LPR>(ss);
    gx = token_sum<LPR>(gx);
    const float rrms = 1.0f / sqrtf((float)(ss / (double)D) + prod.eps);
    const float cr = (float)(gx / (double)D) * rrms * rrms;
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p)
      o[p] = pack_bf16x2(rrms * (gp[2 * p] - x[2 * p] * cr), rrms * (gp[2 * p + 1] - x[2 * p + 1] * cr));
    return make_uint4(o[0], o[1], o[2], o[3]);
  };
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t t = tok0 + rr + ps * RPP;
    const int64_t tok = min(t, n - 1);  // clamped: the lanes of a token reduce together
    const int64_t gofs = ((int64_t)bh * n + tok) * D + c8 * 8;
    const uint4 xq = *reinterpret_cast<const uint4*>(src.q + tok * src.stride + c8 * 8);
    const uint4 xk = *reinterpret_cast<const uint4*>(src.k + tok * src.stride + c8 * 8);
    const uint4 g_q = *reinterpret_cast<const uint4*>(gq + gofs);
    const uint4 g_k = *reinterpret_cast<const uint4*>(gk + gofs);
    const uint4 g_v = *reinterpret_cast<const uint4*>(gv + gofs);
    f32x4 fr[4];
    load_freqs<D>(prod.freqs, src.row0 + tok, c8, fr);
    const uint4 dq = one(xq, g_q, qn, fr);
    const uint4 dk = one(xk, g_k, kn, fr);
    if (t < n) {
      uint16_t* row = dqkv + (src.row0 + t) * 3 * third + head_off + c8 * 8;
      *reinterpret_cast<uint4*>(row) = dq;
      *reinterpret_cast<uint4*>(row + third) = dk;
      *reinterpret_cast<uint4*>(row + 2 * third) = g_v;
    }
  }
}

// Tokens per K column-sum chunk.
constexpr int kSumTokens = 256;

__host__ __device__ inline int64_t k_sum_chunks(int64_t n) { return (n + kSumTokens - 1) / kSumTokens; }

// Smoothing pass 1: fp64 column sums of K over each 256-token chunk of each
// head, part[bh][chunk][d].  One workgroup per (chunk, bh); lane (rr, c8)
// holds channels [8*c8, +8) of tokens rr + RPP*ps.  Every sum is formed in a
// fixed order, so the result does not depend on scheduling.  PROD: K comes
// from the projection output through the producer (RMSNorm + rotary), four
// tokens per lane at a time.
template <int D, bool PROD>
__global__ void __launch_bounds__(256) k_colsum_kernel(const uint16_t* __restrict__ k, int64_t n,
                                                       double* __restrict__ part, ProdArgs prod) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = kSumTokens / RPP;
  constexpr int GROUP = PROD ? 4 : PASSES;  // tokens per lane loaded together
  __shared__ double ksw[4][D];
  int64_t ch;
  int bh;
  block_coords<PROD>(prod, ch, bh);
  const int tid = threadIdx.x, wave = tid >> 6;
  const int c8 = tid % LPR, rr = tid / LPR;
  const int64_t tok0 = (int64_t)ch * kSumTokens;
  const HeadRows<D, PROD> src(k, k, k, prod, bh, n);
  float kn[8];
  if constexpr (PROD) load_w8(prod.kw, c8, kn);
  double cs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) cs[e] = 0.0;
#pragma unroll 1
  for (int g0 = 0; g0 < PASSES; g0 += GROUP) {
    uint4 w[GROUP];
#pragma unroll
    for (int i = 0; i < GROUP; ++i) {
      const int64_t tok = min(tok0 + rr + (g0 + i) * RPP, n - 1);  // clamped in bounds, masked below
      w[i] = *reinterpret_cast<const uint4*>(src.k + tok * src.stride + c8 * 8);
    }
    if constexpr (PROD) {
#pragma unroll
      for (int i = 0; i < GROUP; ++i) {
        f32x4 fr[4];
        load_freqs<D>(prod.freqs, src.row0 + min(tok0 + rr + (g0 + i) * RPP, n - 1), c8, fr);
        w[i] = rms_rope8<D>(w[i], kn, fr, prod.eps);
      }
    }
#pragma unroll
    for (int i = 0; i < GROUP; ++i) {
      float x[8];
      unpack8(w[i], x);
      const bool keep = tok0 + rr + (g0 + i) * RPP < n;
#pragma unroll
      for (int e = 0; e < 8; ++e) cs[e] += keep ? (double)x[e] : 0.0;
    }
  }
  // token rows of the wave (lanes c8 + LPR*m), then the 4 waves
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) cs[e] += __shfl_xor(cs[e], off);
  if ((tid & 63) < LPR) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ksw[wave][c8 * 8 + e] = cs[e];
  }
  __syncthreads();
  if (tid < D)
    part[((int64_t)bh * k_sum_chunks(n) + ch) * D + tid] = (ksw[0][tid] + ksw[1][tid]) + (ksw[2][tid] + ksw[3][tid]);
}

// One workgroup per (64-token block, bh).
//   Q, K: lane (rr, c8) holds channels [8*c8, +8) of tokens rr + RPP*ps.
//   V:    lane (g, c8) holds channels [8*c8, +8) of the 4 consecutive tokens
//         4g..4g+3, so the 4 codes of a channel form one 32-bit fragment word.
// With smoothing, the head's mean is the sum of its chunk sums (fixed order)
// / N in fp64, rounded to fp32 then bf16 (the reference's bf16 mean), and K
// rows are smoothed as bf16(k - mean).  PROD: q, k and v come from the
// projection output, q and k through the producer (RMSNorm + rotary), so the
// codes equal those of the producer's bf16 outputs.
template <int D, int QK, int PV, int GRAN, bool SMOOTH, bool PROD>
__global__ void __launch_bounds__(256) quantize_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    int64_t n, int64_t np, float fold, const double* __restrict__ ksum_part,
    uint8_t* __restrict__ qc, float* __restrict__ qs, uint8_t* __restrict__ kc, float* __restrict__ ks,
    uint8_t* __restrict__ vout, float* __restrict__ vs, uint16_t* __restrict__ kmean, ProdArgs prod) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  constexpr int VTHREADS = 16 * LPR;  // 16 groups of 4 tokens
  __shared__ unsigned int blk_amax[2];
  __shared__ __attribute__((aligned(16))) float vmax[4][D];
  // smoothing: the TPC threads of a column each sum every TPC-th chunk sum
  constexpr int TPC = 256 / D;
  constexpr int kMeanLoads = 12;  // chunk sums in flight per thread
  __shared__ double msum[SMOOTH ? TPC : 1][D];
  __shared__ float mu[SMOOTH ? D : 1];
  // V operand image of this 64-token block in fragment order; written to
  // global as contiguous 16-byte chunks
  __shared__ __attribute__((aligned(16))) uint8_t vimg[(PV == kPV_FP8 ? 1 : 2) * 64 * D];
  int64_t blk;
  int bh;
  block_coords<PROD>(prod, blk, bh);
  const int tid = threadIdx.x, wave = tid >> 6;
  const int c8 = tid % LPR, rr = tid / LPR;
  const int64_t tok0 = (int64_t)blk * 64;
  const HeadRows<D, PROD> src(q, k, v, prod, bh, n);
  const int64_t co = (int64_t)bh * np * D;
  const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);

  if (tid < 2) blk_amax[tid] = 0u;
  __syncthreads();

  // ---- smoothing: this thread's chunk sums, loaded before the block's data ----
  // Thread (j = tid / D, column tid % D) adds chunks j, j + TPC, ... in order.
  const int64_t nch = SMOOTH ? k_sum_chunks(n) : 0;
  const double* pp = ksum_part + ((int64_t)bh * nch + tid / D) * D + tid % D;
  double mt[SMOOTH ? kMeanLoads : 1];
  if constexpr (SMOOTH) {
#pragma unroll
    for (int i = 0; i < kMeanLoads; ++i) mt[i] = tid / D + TPC * i < nch ? pp[(int64_t)TPC * i * D] : 0.0;
  }

  // ---- issue every load of the block up front ------------------------------
  // Token indices are clamped to N-1 so every load is in bounds and issued
  // without branches; values of tokens past N are zeroed afterwards.
  uint4 qw[PASSES], kw[PASSES], vw[4];
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t tok = min(tok0 + rr + ps * RPP, n - 1);
    qw[ps] = *reinterpret_cast<const uint4*>(src.q + tok * src.stride + c8 * 8);
    kw[ps] = *reinterpret_cast<const uint4*>(src.k + tok * src.stride + c8 * 8);
  }
  const int g = (tid / LPR) & 15;  // V token group (V work only for tid < VTHREADS)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t tok = min(tok0 + 4 * g + i, n - 1);
    vw[i] = *reinterpret_cast<const uint4*>(src.v + tok * src.stride + c8 * 8);
  }
  if constexpr (PROD) {
    // the producer's bf16 q and k (every lane of a token takes part in its sum)
    float qn[8], kn[8];
    load_w8(prod.qw, c8, qn);
    load_w8(prod.kw, c8, kn);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      f32x4 fr[4];
      load_freqs<D>(prod.freqs, src.row0 + min(tok0 + rr + ps * RPP, n - 1), c8, fr);
      qw[ps] = rms_rope8<D>(qw[ps], qn, fr, prod.eps);
      kw[ps] = rms_rope8<D>(kw[ps], kn, fr, prod.eps);
    }
  }
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    if (tok0 + rr + ps * RPP >= n) {
      qw[ps] = zero4;
      kw[ps] = zero4;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (tid >= VTHREADS || tok0 + 4 * g + i >= n) vw[i] = zero4;
  if constexpr (SMOOTH) {
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < kMeanLoads; ++i) s += mt[i];
    for (int64_t c = tid / D + TPC * kMeanLoads; c < nch; c += TPC) s += pp[(c - tid / D) * D];  // long heads
    msum[tid / D][tid % D] = s;  // combined after the V section's barrier
  }
  // ---- Q -----------------------------------------------------------------------
  {
    float x[PASSES][8], amax[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) unpack8(qw[ps], x[ps]);
    row_amax<D, GRAN, PASSES>(x, amax, &blk_amax[0]);
    store_rows<D, QK, GRAN, PASSES>(x, amax, tok0, rr, c8, fold, qc + co, qs + sco, tid);
  }

  // ---- V -------------------------------------------------------------------------
  if (PV == kPV_FP8) {
    // channel maxima of |v| over the 4 tokens, on the bf16 bit patterns: for
    // non-NaN values the magnitude bits order like the magnitudes, and the
    // 32 unpacked floats need not stay live across the barrier below
    float cm[8];
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      u16x2 m = __builtin_bit_cast(u16x2, word_of(vw[0], w4) & 0x7fff7fffu);
#pragma unroll
      for (int i = 1; i < 4; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, word_of(vw[i], w4) & 0x7fff7fffu));
      cm[2 * w4] = __uint_as_float((uint32_t)m.x << 16);
      cm[2 * w4 + 1] = __uint_as_float((uint32_t)m.y << 16);
    }
    // across the token groups of this wave (lanes c8 + LPR*m), then across waves
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (LPR == 8) {
        cm[e] = fmaxf(cm[e], __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(cm[e]), 0x128, 0xf, 0xf, false)));  // row_ror:8
      }
      cm[e] = rows_max(cm[e]);
    }
    if (tid < VTHREADS && (tid & 63) < LPR) {
#pragma unroll
      for (int e = 0; e < 8; ++e) vmax[wave][c8 * 8 + e] = cm[e];
    }
    __syncthreads();
    constexpr int VW = VTHREADS / 64;  // waves holding V
    if (tid < VTHREADS) {
      float am[8];
      {
        const f32x4* v4 = reinterpret_cast<const f32x4*>(&vmax[0][c8 * 8]);
        const f32x4 a0 = v4[0], a1 = v4[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          am[i] = a0[i];
          am[4 + i] = a1[i];
        }
#pragma unroll
        for (int ww = 1; ww < VW; ++ww) {
          const f32x4* w4 = reinterpret_cast<const f32x4*>(&vmax[ww][c8 * 8]);
          const f32x4 b0 = w4[0], b1 = w4[1];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            am[i] = fmaxf(am[i], b0[i]);
            am[4 + i] = fmaxf(am[4 + i], b1[i]);
          }
        }
      }
      float inv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) inv[e] = kFp8Max / fmaxf(am[e], kEps);
      if (g == 0) {
        f32x4* o4 = reinterpret_cast<f32x4*>(vs + ((int64_t)bh * (np / 64) + blk) * D + c8 * 8);
        o4[0] = f32x4{am[0] / kFp8Max, am[1] / kFp8Max, am[2] / kFp8Max, am[3] / kFp8Max};
        o4[1] = f32x4{am[4] / kFp8Max, am[5] / kFp8Max, am[6] / kFp8Max, am[7] / kFp8Max};
      }
      // word of channel d = 32j + r for tokens 4g..4g+3 -> chunk (j, b, L = 32h + r), byte 4jj,
      // with g = 8b + 2jj + h
      const int b = g >> 3, jj = (g >> 1) & 3, hh = g & 1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = c8 * 8 + e, j = d >> 5, r = d & 31;
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = word_of(vw[i], e >> 1);
          x[i] = __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
        }
        const uint32_t word = pack_fp8x4(x[0] * inv[e], x[1] * inv[e], x[2] * inv[e], x[3] * inv[e]);
        *reinterpret_cast<uint32_t*>(vimg + (((j * 2 + b) * 64 + 32 * hh + r) * 16) + 4 * jj) = word;
      }
    }
  } else if (tid < VTHREADS) {
    // bf16 V: element 4jj + i of chunk (j, b, tt, L) = V[32b + 16tt + 8jj + 4h + i][32j + r],
    // with g = 8b + 4tt + 2jj + h
    const int b = g >> 3, tt = (g >> 2) & 1, jj = (g >> 1) & 1, hh = g & 1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = c8 * 8 + e, j = d >> 5, r = d & 31;
      const int sh = (e & 1) * 16;
      uint32_t t4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) t4[i] = (word_of(vw[i], e >> 1) >> sh) & 0xffffu;
      uint2 pk;
      pk.x = t4[0] | (t4[1] << 16);
      pk.y = t4[2] | (t4[3] << 16);
      *reinterpret_cast<uint2*>(vimg + (((((j * 2 + b) * 2 + tt) * 64 + 32 * hh + r) * 8) + 4 * jj) * 2) = pk;
    }
  }
  __syncthreads();
  if constexpr (SMOOTH) {
    if (tid < D) {
      double s = msum[0][tid];
#pragma unroll
      for (int j = 1; j < TPC; ++j) s += msum[j][tid];
      const uint16_t m16 = f32_to_bf16_rne((float)(s / (double)n));
      mu[tid] = bf16_to_f32(m16);
      if (blk == 0) kmean[(int64_t)bh * D + tid] = m16;
    }
  }
  {
    constexpr int VBYTES = (PV == kPV_FP8 ? 1 : 2) * 64 * D;
    uint8_t* vo = vout + (PV == kPV_FP8 ? 1 : 2) * (co + tok0 * D);
#pragma unroll
    for (int i = tid; i < VBYTES / 16; i += 256)
      reinterpret_cast<uint4*>(vo)[i] = reinterpret_cast<const uint4*>(vimg)[i];
  }
  if constexpr (SMOOTH) __syncthreads();  // mu

  // ---- K ---------------------------------------------------------------------
  {
    float x[PASSES][8], amax[PASSES];
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      unpack8(kw[ps], x[ps]);
      if constexpr (SMOOTH) {
        // rows past N were loaded as zeros; keep them zero after the shift
        const float keep = tok0 + rr + ps * RPP < n ? 1.0f : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[ps][e] = bf16_to_f32(f32_to_bf16_rne(x[ps][e] - mu[c8 * 8 + e])) * keep;
      }
    }
    row_amax<D, GRAN, PASSES>(x, amax, &blk_amax[1]);
    store_rows<D, QK, GRAN, PASSES>(x, amax, tok0, rr, c8, 1.0f, kc + co, ks + sco, tid);
  }
}

// Arguments of one quantization call.
struct QuantCall {
  const uint16_t *q, *k, *v;
  int64_t bh, n;
  float fold;
  double* ws;
  uint8_t* qc;
  float* qs;
  uint8_t* kc;
  float* ks;
  uint8_t* vout;
  float* vs;
  uint16_t* kmean;
  ProdArgs prod;
};

template <int D, int QK, int PV, int GRAN, bool SMOOTH, bool PROD>
hipError_t launch_quantize_t(const QuantCall& a, hipStream_t st) {
  const int64_t np = padded_len(a.n);
  const int nblk = (int)(np / 64);
  if (SMOOTH) {
    const int64_t nch = k_sum_chunks(a.n);
    const dim3 g = PROD ? dim3((unsigned)(nch * a.bh)) : dim3((unsigned)nch, (unsigned)a.bh);
    hipLaunchKernelGGL((k_colsum_kernel<D, PROD>), g, dim3(256), 0, st, a.k, a.n, a.ws, a.prod);
  }
  const dim3 grid = PROD ? dim3((unsigned)((int64_t)nblk * a.bh)) : dim3((unsigned)nblk, (unsigned)a.bh);
  hipLaunchKernelGGL((quantize_kernel<D, QK, PV, GRAN, SMOOTH, PROD>), grid, dim3(256), 0, st, a.q, a.k, a.v, a.n, np, a.fold, a.ws, a.qc, a.qs, a.kc, a.ks, a.vout, a.vs,
                     a.kmean, a.prod);
  return hipGetLastError();
}

template <int D, int QK, int PV, int GRAN>
hipError_t launch_quantize_s(bool smooth, const QuantCall& a, hipStream_t st) {
  const bool prod = a.prod.qkv != nullptr;
  if (smooth)
    return prod ? launch_quantize_t<D, QK, PV, GRAN, true, true>(a, st)
                : launch_quantize_t<D, QK, PV, GRAN, true, false>(a, st);
  return prod ? launch_quantize_t<D, QK, PV, GRAN, false, true>(a, st)
              : launch_quantize_t<D, QK, PV, GRAN, false, false>(a, st);
}

template <int D>
hipError_t launch_quantize_d(int qk, int pv, int gran, bool smooth, const QuantCall& a, hipStream_t st) {
#define SAGE_Q_CASE(QK_, PV_, G_) \
  if (qk == QK_ && pv == PV_ && gran == G_) return launch_quantize_s<D, QK_, PV_, G_>(smooth, a, st);
  SAGE_Q_CASE(0, 0, 0) SAGE_Q_CASE(0, 0, 1) SAGE_Q_CASE(0, 1, 0) SAGE_Q_CASE(0, 1, 1)
  SAGE_Q_CASE(1, 0, 0) SAGE_Q_CASE(1, 0, 1) SAGE_Q_CASE(1, 1, 0) SAGE_Q_CASE(1, 1, 1)
#undef SAGE_Q_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_quantize(int qk, int pv, int gran, bool smooth, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, int64_t bh, int64_t n, int64_t d, float fold, double* ws,
                           uint8_t* qc, float* qs, uint8_t* kc, float* ks, uint8_t* vout, float* vs,
                           uint16_t* kmean, const ProdArgs& prod, hipStream_t st) {
  const QuantCall a{q, k, v, bh, n, fold, ws, qc, qs, kc, ks, vout, vs, kmean, prod};
  if (d == 128) return launch_quantize_d<128>(qk, pv, gran, smooth, a, st);
  if (d == 64) return launch_quantize_d<64>(qk, pv, gran, smooth, a, st);
  return hipErrorInvalidValue;
}

hipError_t launch_qkv_postprocess(const ProdArgs& prod, int64_t bh, int64_t n, int64_t d, uint16_t* q_out,
                                  uint16_t* k_out, uint16_t* v_out, hipStream_t st) {
  const dim3 grid((unsigned)((n + 63) / 64 * bh));  // head fastest (block_coords)
  if (d == 128)
    hipLaunchKernelGGL(qkv_postprocess_kernel<128>, grid, dim3(256), 0, st, prod, n, q_out, k_out, v_out);
  else if (d == 64)
    hipLaunchKernelGGL(qkv_postprocess_kernel<64>, grid, dim3(256), 0, st, prod, n, q_out, k_out, v_out);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_qkv_postprocess_bwd(const ProdArgs& prod, int64_t bh, int64_t n, int64_t d, const uint16_t* gq,
                                      const uint16_t* gk, const uint16_t* gv, uint16_t* dqkv, hipStream_t st) {
  const dim3 grid((unsigned)((n + 63) / 64 * bh));  // head fastest (block_coords)
  if (d == 128)
    hipLaunchKernelGGL(qkv_postprocess_bwd_kernel<128>, grid, dim3(256), 0, st, prod, n, gq, gk, gv, dqkv);
  else if (d == 64)
    hipLaunchKernelGGL(qkv_postprocess_bwd_kernel<64>, grid, dim3(256), 0, st, prod, n, gq, gk, gv, dqkv);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// fp64 column sums of K per head and 256-token chunk, [bh][ceil(n/256)][d].
size_t quant_workspace_bytes(int64_t bh, int64_t n, int64_t d) {
  return (size_t)(bh * k_sum_chunks(n) * d) * sizeof(double);
}

}  // namespace sage
