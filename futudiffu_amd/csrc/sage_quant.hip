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
#include "sage_common.h"
#include "sage_launch.h"

namespace sage {

constexpr int kSumChunk = 256;  // tokens per partial K column sum

// Pass 1: fp64 partial column sums of K per (bh, 256-token chunk).
// The sum of bf16 values in fp64 is exact for realistic inputs, so the mean
// does not depend on the order the chunks are combined in.
template <int D>
__global__ void __launch_bounds__(256) k_colsum_kernel(const uint16_t* __restrict__ k, int64_t n,
                                                       double* __restrict__ ws, int nchunks) {
  constexpr int LPR = D / 8;       // lanes per token row (8 channels each)
  constexpr int RPP = 256 / LPR;   // rows per pass
  __shared__ double red[RPP * D];
  const int bh = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
  const int c8 = tid % LPR, rr = tid / LPR;
  const uint16_t* kb = k + (int64_t)bh * n * D;
  double acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0;
  const int64_t r0 = (int64_t)chunk * kSumChunk;
  const int64_t r1 = r0 + kSumChunk < n ? r0 + kSumChunk : n;
  for (int64_t r = r0 + rr; r < r1; r += RPP) {
    const uint4 w = *reinterpret_cast<const uint4*>(kb + r * D + c8 * 8);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] += (double)bf16_to_f32((uint16_t)(ww[e] & 0xffffu));
      acc[2 * e + 1] += (double)bf16_to_f32((uint16_t)(ww[e] >> 16));
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[rr * D + c8 * 8 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    double s = 0.0;
    for (int i = 0; i < RPP; ++i) s += red[i * D + tid];
    ws[((int64_t)bh * nchunks + chunk) * D + tid] = s;
  }
}

// Load 8 bf16 channels [8*c8, 8*c8+8) of token `tok` as fp32 (zeros past n).
template <int D>
__device__ __forceinline__ void load8(const uint16_t* __restrict__ base, int64_t tok, int64_t n, int c8,
                                      float x[8]) {
  if (tok < n) {
    const uint4 w = *reinterpret_cast<const uint4*>(base + tok * D + c8 * 8);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf16_to_f32((uint16_t)(ww[e] & 0xffffu));
      x[2 * e + 1] = bf16_to_f32((uint16_t)(ww[e] >> 16));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = 0.0f;
  }
}

// Quantize one operand (Q or K) for the 64 tokens of this workgroup and write
// codes in row-fragment order plus scales.
template <int D, int QK, int GRAN, bool SMOOTH>
__device__ __forceinline__ void quantize_rows(const uint16_t* __restrict__ src, int64_t n, int64_t np,
                                              int64_t tok0, const float* mu, float fold,
                                              uint8_t* __restrict__ codes, float* __restrict__ scale,
                                              unsigned int* blk_amax_u) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  const int tid = threadIdx.x, c8 = tid % LPR, rr = tid / LPR;
  const float qmax = (QK == kQK_INT8) ? kInt8Max : kFp8Max;
  float x[PASSES][8];
  float ramax[PASSES];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t tok = tok0 + rr + ps * RPP;
    load8<D>(src, tok, n, c8, x[ps]);
    if (SMOOTH && tok < n) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[ps][e] = bf16_to_f32(f32_to_bf16_rne(x[ps][e] - mu[c8 * 8 + e]));
    }
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) a = fmaxf(a, fabsf(x[ps][e]));
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) a = fmaxf(a, __shfl_xor(a, off, LPR));
    ramax[ps] = a;
  }
  if (GRAN == kGRAN_BLOCK64) {
    float a = 0.0f;
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) a = fmaxf(a, ramax[ps]);
    if (c8 == 0) atomicMax(blk_amax_u, __float_as_uint(a));
    __syncthreads();
    a = __uint_as_float(*blk_amax_u);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) ramax[ps] = a;
  }
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t tok = tok0 + rr + ps * RPP;
    const float amax = ramax[ps];
    const float inv = qmax / fmaxf(amax, kEps);  // IEEE division (correctly rounded)
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
    const int64_t off = row_frag_offset(tok, d0 / 32, (d0 / 16) & 1, D) + (d0 & 8);
    *reinterpret_cast<uint2*>(codes + off) = word;
    if (GRAN == kGRAN_TOKEN) {
      if (c8 == 0) scale[tok] = (amax / qmax) * fold;
    } else if (tid == 0 && ps == 0) {
      scale[tok0 / 64] = (amax / qmax) * fold;
    }
  }
}

// Pass 2: one workgroup per (64-token block, bh).
template <int D, int QK, int PV, int GRAN, bool SMOOTH>
__global__ void __launch_bounds__(256) quantize_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    int64_t n, int64_t np, float fold, const double* __restrict__ ws, int nchunks,
    uint8_t* __restrict__ qc, float* __restrict__ qs, uint8_t* __restrict__ kc, float* __restrict__ ks,
    uint8_t* __restrict__ vout, float* __restrict__ vs, uint16_t* __restrict__ kmean) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  __shared__ float mu[D];
  __shared__ unsigned int amax_u[2 + D];
  __shared__ __attribute__((aligned(16))) uint8_t vt[(PV == kPV_FP8 ? 1 : 2) * 64 * D];
  const int bh = blockIdx.y, blk = blockIdx.x, tid = threadIdx.x;
  const int64_t tok0 = (int64_t)blk * 64;
  if (tid < 2 + D) amax_u[tid] = 0u;
  if (SMOOTH && tid < D) {
    double s = 0.0;
    for (int c = 0; c < nchunks; ++c) s += ws[((int64_t)bh * nchunks + c) * D + tid];
    const uint16_t m16 = f32_to_bf16_rne((float)(s / (double)n));
    mu[tid] = bf16_to_f32(m16);
    if (blk == 0) kmean[(int64_t)bh * D + tid] = m16;
  }
  __syncthreads();
  const int64_t so = (int64_t)bh * n * D;
  const int64_t co = (int64_t)bh * np * D;
  const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);
  quantize_rows<D, QK, GRAN, false>(q + so, n, np, tok0, mu, fold, qc + co, qs + sco, &amax_u[0]);
  quantize_rows<D, QK, GRAN, SMOOTH>(k + so, n, np, tok0, mu, 1.0f, kc + co, ks + sco, &amax_u[1]);

  // V: stage this 64-token tile in LDS, then write the transposed fragments.
  const int c8 = tid % LPR, rr = tid / LPR;
  if (PV == kPV_FP8) {
    float x[PASSES][8];
    float cm[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) cm[e] = 0.0f;
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      load8<D>(v + so, tok0 + rr + ps * RPP, n, c8, x[ps]);
#pragma unroll
      for (int e = 0; e < 8; ++e) cm[e] = fmaxf(cm[e], fabsf(x[ps][e]));
    }
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e) cm[e] = fmaxf(cm[e], __shfl_xor(cm[e], off));
    if ((tid & 63) < LPR) {
#pragma unroll
      for (int e = 0; e < 8; ++e) atomicMax(&amax_u[2 + c8 * 8 + e], __float_as_uint(cm[e]));
    }
    __syncthreads();
    float inv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) inv[e] = kFp8Max / fmaxf(__uint_as_float(amax_u[2 + c8 * 8 + e]), kEps);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = rr + ps * RPP;
      uint2 word;
      word.x = pack_fp8x4(x[ps][0] * inv[0], x[ps][1] * inv[1], x[ps][2] * inv[2], x[ps][3] * inv[3]);
      word.y = pack_fp8x4(x[ps][4] * inv[4], x[ps][5] * inv[5], x[ps][6] * inv[6], x[ps][7] * inv[7]);
      *reinterpret_cast<uint2*>(vt + row * D + c8 * 8) = word;
    }
    if (tid < D) vs[((int64_t)bh * (np / 64) + blk) * D + tid] = __uint_as_float(amax_u[2 + tid]) / kFp8Max;
    __syncthreads();
    // 16-byte chunk (j, b, L): byte 4*jj + i = Vc[32b + 8jj + 4h + i][32j + r]
    constexpr int CHUNKS = (D / 32) * 2 * 64;
    uint8_t* vo = vout + co + tok0 * D;
    for (int ch = tid; ch < CHUNKS; ch += 256) {
      const int L = ch & 63, b = (ch >> 6) & 1, j = ch >> 7;
      const int h = L >> 5, r = L & 31, d = 32 * j + r;
      uint32_t w4[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int key = 32 * b + 8 * jj + 4 * h;
        w4[jj] = (uint32_t)vt[(key + 0) * D + d] | ((uint32_t)vt[(key + 1) * D + d] << 8) |
                 ((uint32_t)vt[(key + 2) * D + d] << 16) | ((uint32_t)vt[(key + 3) * D + d] << 24);
      }
      *reinterpret_cast<uint4*>(vo + (int64_t)ch * 16) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
  } else {
    uint16_t* vt16 = reinterpret_cast<uint16_t*>(vt);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      const int row = rr + ps * RPP;
      const int64_t tok = tok0 + row;
      uint4 w = make_uint4(0, 0, 0, 0);
      if (tok < n) w = *reinterpret_cast<const uint4*>(v + so + tok * D + c8 * 8);
      *reinterpret_cast<uint4*>(vt16 + row * D + c8 * 8) = w;
    }
    __syncthreads();
    // 16-byte chunk (j, b, tt, L): element 4*jj + i = V[32b + 16tt + 8jj + 4h + i][32j + r]
    constexpr int CHUNKS = (D / 32) * 4 * 64;
    uint8_t* vo = vout + 2 * (co + tok0 * D);
    for (int ch = tid; ch < CHUNKS; ch += 256) {
      const int L = ch & 63, tt = (ch >> 6) & 1, b = (ch >> 7) & 1, j = ch >> 8;
      const int h = L >> 5, r = L & 31, d = 32 * j + r;
      uint32_t w4[4];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int key = 32 * b + 16 * tt + 8 * jj + 4 * h;
        w4[2 * jj] = (uint32_t)vt16[(key + 0) * D + d] | ((uint32_t)vt16[(key + 1) * D + d] << 16);
        w4[2 * jj + 1] = (uint32_t)vt16[(key + 2) * D + d] | ((uint32_t)vt16[(key + 3) * D + d] << 16);
      }
      *reinterpret_cast<uint4*>(vo + (int64_t)ch * 16) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
  }
}

template <int D, int QK, int PV, int GRAN, bool SMOOTH>
hipError_t launch_quantize_t(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t bh, int64_t n,
                             float fold, double* ws, uint8_t* qc, float* qs, uint8_t* kc, float* ks,
                             uint8_t* vout, float* vs, uint16_t* kmean, hipStream_t st) {
  const int64_t np = padded_len(n);
  const int nchunks = (int)((n + kSumChunk - 1) / kSumChunk);
  if (SMOOTH) {
    hipLaunchKernelGGL((k_colsum_kernel<D>), dim3(nchunks, (unsigned)bh), dim3(256), 0, st, k, n, ws, nchunks);
  }
  hipLaunchKernelGGL((quantize_kernel<D, QK, PV, GRAN, SMOOTH>), dim3((unsigned)(np / 64), (unsigned)bh),
                     dim3(256), 0, st, q, k, v, n, np, fold, ws, nchunks, qc, qs, kc, ks, vout, vs, kmean);
  return hipGetLastError();
}

template <int D, int QK, int PV, int GRAN>
hipError_t launch_quantize_s(bool smooth, const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t bh,
                             int64_t n, float fold, double* ws, uint8_t* qc, float* qs, uint8_t* kc, float* ks,
                             uint8_t* vout, float* vs, uint16_t* kmean, hipStream_t st) {
  return smooth ? launch_quantize_t<D, QK, PV, GRAN, true>(q, k, v, bh, n, fold, ws, qc, qs, kc, ks, vout, vs,
                                                           kmean, st)
                : launch_quantize_t<D, QK, PV, GRAN, false>(q, k, v, bh, n, fold, ws, qc, qs, kc, ks, vout,
                                                            vs, kmean, st);
}

template <int D>
hipError_t launch_quantize_d(int qk, int pv, int gran, bool smooth, const uint16_t* q, const uint16_t* k,
                             const uint16_t* v, int64_t bh, int64_t n, float fold, double* ws, uint8_t* qc,
                             float* qs, uint8_t* kc, float* ks, uint8_t* vout, float* vs, uint16_t* kmean,
                             hipStream_t st) {
#define SAGE_Q_CASE(QK_, PV_, G_)                                                                        \
  if (qk == QK_ && pv == PV_ && gran == G_)                                                              \
    return launch_quantize_s<D, QK_, PV_, G_>(smooth, q, k, v, bh, n, fold, ws, qc, qs, kc, ks, vout, vs, \
                                              kmean, st);
  SAGE_Q_CASE(0, 0, 0) SAGE_Q_CASE(0, 0, 1) SAGE_Q_CASE(0, 1, 0) SAGE_Q_CASE(0, 1, 1)
  SAGE_Q_CASE(1, 0, 0) SAGE_Q_CASE(1, 0, 1) SAGE_Q_CASE(1, 1, 0) SAGE_Q_CASE(1, 1, 1)
#undef SAGE_Q_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_quantize(int qk, int pv, int gran, bool smooth, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, int64_t bh, int64_t n, int64_t d, float fold, double* ws,
                           uint8_t* qc, float* qs, uint8_t* kc, float* ks, uint8_t* vout, float* vs,
                           uint16_t* kmean, hipStream_t st) {
  if (d == 128)
    return launch_quantize_d<128>(qk, pv, gran, smooth, q, k, v, bh, n, fold, ws, qc, qs, kc, ks, vout, vs, kmean,
                                  st);
  if (d == 64)
    return launch_quantize_d<64>(qk, pv, gran, smooth, q, k, v, bh, n, fold, ws, qc, qs, kc, ks, vout, vs, kmean,
                                 st);
  return hipErrorInvalidValue;
}

size_t quant_workspace_bytes(int64_t bh, int64_t n, int64_t d) {
  const int64_t nchunks = (n + kSumChunk - 1) / kSumChunk;
  return (size_t)(bh * nchunks * d) * sizeof(double);
}

}  // namespace sage
