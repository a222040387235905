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
// Every workgroup has one role: the fp64 column sums of one K chunk (for the
// smoothing mean), or the Q, V or K codes of one 64-token block of one head.
// Rows past N are read through buffer resources, which return zeros.  With
// smoothing the mean makes a second read of K unavoidable (every K code
// depends on all N tokens); one kernel (quantize_one_kernel) dispatches the
// column sums first and the K blocks last, which wait for their head's sums
// through flags tagged with a per-call epoch.  Under stream capture the
// launch uses two kernels instead (quantize_qv_kernel, quantize_k_kernel):
// a captured epoch would repeat on every replay.  Both forms write the same
// bits.
#include "sage_common.h"
#include "sage_launch.h"

#include <atomic>
#include <chrono>
#include <cstdlib>
#include <cstring>

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
// The operands are non-negative and not NaN, so their bit patterns order like
// their values: an integer max fuses with the permute into one instruction.
template <int G>
__device__ __forceinline__ float group_max(float a) {
  uint32_t u = __float_as_uint(a);
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xf, 0xf, true));   // [1,0,3,2]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x4E, 0xf, 0xf, true));   // [2,3,0,1]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x141, 0xf, 0xf, true));  // half mirror
  if constexpr (G == 16) u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x140, 0xf, 0xf, true));
  return __uint_as_float(u);
}

// Max across the 16-lane rows of a wave (lanes l, l^16, l^32, l^48), for
// non-negative, non-NaN operands (integer max of the bit patterns).
__device__ __forceinline__ float rows_max(float a) {
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
  const uint32_t m = max((uint32_t)s16[0], (uint32_t)s16[1]);
  const auto s32 = __builtin_amdgcn_permlane32_swap(m, m, false, false);
  return __uint_as_float(max((uint32_t)s32[0], (uint32_t)s32[1]));
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t word_of(uint4 w, int i) {
  return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
}

// Lane p of each quad, broadcast to the quad (p a constant after unrolling).
template <int P>
__device__ __forceinline__ float quad_lane_c(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), P * 0x55, 0xf, 0xf, true));
}
__device__ __forceinline__ float quad_lane(float x, int p) {
  return p == 0 ? quad_lane_c<0>(x) : p == 1 ? quad_lane_c<1>(x) : p == 2 ? quad_lane_c<2>(x) : quad_lane_c<3>(x);
}

// Quantize the 8 channels a lane holds for each of its PASSES tokens of one
// operand (Q or K) and store codes in row-fragment order plus scales.
// x holds the (smoothed) values; amax is per token, or per 64-token block, and
// the same in every lane of a token.  The correctly rounded divisions
// qmax / amax and amax / qmax are formed once per quad: lane c8 (mod 4) works
// for pass c8 % PASSES, and a quad permute hands every lane the result of
// each pass.  Lane c8 = ps stores token ps's scale.
template <int D, int QK, int GRAN, int PASSES>
__device__ __forceinline__ void store_rows(const float (&x)[PASSES][8], const float (&amax)[PASSES], int64_t tok0,
                                           int rr, int c8, float fold, uint8_t* __restrict__ codes,
                                           float* __restrict__ scale, int tid) {
  constexpr int RPP = 256 / (D / 8);
  static_assert(PASSES == 2 || PASSES == 4, "passes per quad");
  const float qmax = (QK == kQK_INT8) ? kInt8Max : kFp8Max;
  // this lane's pass, selected with bit masks (a select chain would become
  // an indexed array in LDS)
  const int mine = c8 & (PASSES - 1);
  uint32_t amb = 0u;
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) amb |= __float_as_uint(amax[ps]) & (0u - (uint32_t)(mine == ps));
  const float am = __uint_as_float(amb);
  const float inv_mine = qmax / fmaxf(am, kEps);  // IEEE division (correctly rounded)
  const float scale_mine = (am / qmax) * fold;
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t tok = tok0 + rr + ps * RPP;
    const float inv = quad_lane(inv_mine, ps);
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
      if (c8 == ps) scale[tok] = scale_mine;
    } else if (tid == 0 && ps == 0) {
      scale[tok0 / 64] = scale_mine;
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

// Slab units (kSlabHeads, sage_launch.h): a workgroup that takes one pass of
// tokens for kSlabHeads heads of a batch (the last group of a batch may have
// fewer) loads the tokens' rotation rows once for all of them.  The rotations
// are 16 bytes per channel pair and token, four times the bf16 data of a
// head; read per head they made up most of the L2 traffic of the
// producer-fused quantization.

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

// Reciprocal RMS of the G tokens (G = 2 or 4) of which a lane holds channels
// [8*c8, +8) (w[g]: token g), rrms = 1 / sqrt(mean(x^2) + eps) over each
// token's D channels (fused_kernels.py:316-320), returned in every lane of a
// quad: lane p of the quad (p < G) holds token p's, so quad_lane_c<g> hands
// every lane token g's.  The sum of squares is formed in fp64 in a fixed
// order: each lane's 8 channels left to right (the squares are exact), then a
// pairwise tree over the token's LPR lanes: lanes l and l^1, then l and l^2
// (quad sums), then quads q and q^1, then (LPR 16) half-rows; rounded once to
// fp32.  The tree is reduce-scattered over the G tokens: at its first level a
// lane keeps tokens {b0, b0 + 2} (b0 = lane bit 0) and hands the other two to
// its partner, at the second it keeps token b0 + 2*b1, so the two levels cost
// G/2 + 1 adds instead of 2G; the quad levels run on the one token left
// (rotating quad r onto r+1 leaves the pair sums in quads 1 and 3 of each
// 16-lane row).  Then one correctly rounded sqrt and division per lane
// instead of one per token, and the results of quads 1 and 3 are copied to
// quads 0 and 2.  fp64 addition is commutative, so every token's sum is the
// same tree's, bit for bit, whichever lane forms it.
template <int D, int G>
__device__ __forceinline__ float tokens_rrms(const uint4 (&w)[G], float eps, int tid) {
  static_assert(G == 2 || G == 4, "tokens per lane");
  constexpr int LPR = D / 8;
  double ss[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float x[8];
    unpack8(w[g], x);
    ss[g] = 0.0;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss[g] = __builtin_fma((double)x[e], (double)x[e], ss[g]);
  }
  const bool b0 = tid & 1, b1 = tid & 2;
  double s;
  if constexpr (G == 4) {
    // lanes l, l^1: keep tokens b0 and b0 + 2, hand over b0^1 and (b0^1) + 2
    const double a0 = (b0 ? ss[1] : ss[0]) + dpp_f64<0xB1>(b0 ? ss[0] : ss[1]);
    const double a2 = (b0 ? ss[3] : ss[2]) + dpp_f64<0xB1>(b0 ? ss[2] : ss[3]);
    // lanes l, l^2: keep token b0 + 2*b1
    s = (b1 ? a2 : a0) + dpp_f64<0x4E>(b1 ? a0 : a2);
  } else {
    s = (b0 ? ss[1] : ss[0]) + dpp_f64<0xB1>(b0 ? ss[0] : ss[1]);  // keep token b0
    s += dpp_f64<0x4E>(s);
  }
  // quads q and q^1 of the token: quad r reads quad r - 1 (row_ror:4), valid
  // in quads 1 and 3; LPR 16: half-rows (row_ror:8), valid in quads 1 and 3
  s += dpp_f64<0x124>(s);
  if constexpr (LPR == 16) s += dpp_f64<0x128>(s);
  const float ms = (float)(s / (double)D);
  float r = 1.0f / sqrtf(ms + eps);  // correctly rounded sqrt and division
  // quads 0 and 2 (banks 0 and 2) take the next quad's (row_shl:4)
  r = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(r), __float_as_int(r), 0x104, 0xf, 0x5, false));
  return r;
}

// RMSNorm + rotary embedding of the 8 channels [8*c8, +8) of one token held
// by a lane (bf16 in, bf16 out), with the token's rrms (tokens_rrms):
// n = x * rrms * w (fused_kernels.py:357-360), and per channel pair (2p, 2p+1)
// with fr[p] = (cos, -sin, sin) (:334-336): even' = cos*n_even + (-sin)*n_odd,
// odd' = sin*n_even + cos*n_odd (:363-366), every product and sum a separately
// rounded fp32 operation.
__device__ __forceinline__ uint4 rope8(uint4 w, float rrms, const float (&nw)[8], const f32x4 (&fr)[4]) {
#pragma clang fp contract(off)  // no fused multiply-add: every product and sum rounds on its own
  float x[8];
  unpack8(w, x);
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
// workgroup per (pass of RPP tokens, group of kSlabHeads heads of a batch),
// groups fastest; lane (rr, c8) holds channels [8*c8, +8) of token s0 + rr,
// loads the token's rotations once and applies them to every head of the
// group, four heads at a time (one reduce-scattered RMS for the four).
template <int D>
__global__ void __launch_bounds__(256) qkv_postprocess_kernel(ProdArgs prod, int64_t n, uint16_t* __restrict__ q_out,
                                                              uint16_t* __restrict__ k_out,
                                                              uint16_t* __restrict__ v_out) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  const int tid = threadIdx.x;
  const int c8 = tid % LPR, rr = tid / LPR;
  const int64_t ngb = (prod.h + kSlabHeads - 1) / kSlabHeads, nsl = (n + RPP - 1) / RPP;
  const int64_t unit = blockIdx.x;
  const int64_t bs = unit / ngb;  // b * nsl + slab
  const int b = (int)(bs / nsl);
  const int64_t s0 = (bs - (int64_t)b * nsl) * RPP;
  const int h0 = (int)(unit - bs * ngb) * kSlabHeads, h1 = min(h0 + kSlabHeads, prod.h);
  const int64_t t = s0 + rr;
  const bool valid = t < n;
  const int64_t tc = valid ? t : n - 1;  // clamped: the lanes of a token reduce together
  f32x4 fr[4];
  load_freqs<D>(prod.freqs, (int64_t)b * n + tc, c8, fr);
  const int64_t hd = (int64_t)prod.h * D;
  const uint16_t* row = prod.qkv + ((int64_t)b * n + tc) * 3 * hd + c8 * 8;
#pragma unroll
  for (int it = 0; it < kSlabHeads / 4; ++it) {
    const int hb = h0 + 4 * it;
    if (hb >= h1) break;  // uniform
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      uint16_t* out = m == 0 ? q_out : m == 1 ? k_out : v_out;
      uint4 w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const uint4*>(row + m * hd + (int64_t)min(hb + j, h1 - 1) * D);
      if (m < 2) {
        const float r = tokens_rrms<D, 4>(w, prod.eps, tid);
        float nw[8];
        load_w8(m == 0 ? prod.qw : prod.kw, c8, nw);
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = rope8(w[j], quad_lane(r, j), nw, fr);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (valid && hb + j < h1)
          *reinterpret_cast<uint4*>(out + (((int64_t)b * prod.h + hb + j) * n + t) * D + c8 * 8) = w[j];
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

// K column sums: each head's tokens form at most kMaxChunks(D) chunks of a
// multiple of 256 tokens, so the quantization reads every chunk sum of a head
// in one round of loads (kMeanLoads per thread, 256 / D threads per channel).
constexpr int kMeanLoads = 12;
__host__ __device__ constexpr int k_max_chunks(int64_t d) { return kMeanLoads * (int)(256 / d); }
__host__ __device__ inline int64_t k_sum_tokens(int64_t n, int64_t d) {
  const int64_t c256 = (n + 255) / 256;
  return 256 * ((c256 + k_max_chunks(d) - 1) / k_max_chunks(d));
}
__host__ __device__ inline int64_t k_sum_chunks(int64_t n, int64_t d) {
  const int64_t t = k_sum_tokens(n, d);
  return (n + t - 1) / t;
}

// Buffer resource over rows [tok0, tok0 + rows) of one head's source (tokens
// `stride` elements apart, D channels each).  Loads past the last valid row
// return zeros, so tokens past N need neither clamping nor masking.
template <int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const uint16_t* src, int64_t stride, int64_t tok0,
                                                            int64_t n, int rows) {
  const int64_t nv = min((int64_t)rows, n - tok0);
  const uint32_t bytes = nv > 0 ? (uint32_t)(((nv - 1) * stride + D) * 2) : 0u;
  return raw_rsrc(src + tok0 * stride, bytes);
}

// 16 bytes at byte offset voff (whole offset in the VGPR: the range check
// covers it), zeros when out of range.
__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t rs, uint32_t voff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voff, 0, 0));
}

// LDS of the quantization workgroups, one role at a time (byte offsets).
template <int D, int PV>
struct QuantLds {
  static constexpr int kVmax = 0;                  // float [4][D]: V channel maxima per wave
  static constexpr int kInv = kVmax + 4 * D * 4;   // float [D]: V inverse scales
  static constexpr int kImg = kInv + D * 4;        // V operand image of the block
  static constexpr int kBytes = kImg + (PV == kPV_FP8 ? 1 : 2) * 64 * D;
  // K column sums: double [4][D] from offset 0; Q/K block amax: 2 words at the end
  static constexpr int kAmax = kBytes;
  static constexpr int kTotal = kAmax + 16;
  static_assert(4 * D * 8 <= kBytes, "column-sum scratch fits");
};

// Issue the 16-byte loads of a lane's tokens of one 64-token block: lane
// (rr, c8) holds channels [8*c8, +8) of tokens rr + RPP*ps.  Rows past N read
// as zeros.
template <int D>
__device__ __forceinline__ void rows_load(const uint16_t* src, int64_t stride, int64_t tok0, int64_t n, int tid,
                                          uint4 (&w)[64 / (256 / (D / 8))]) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  const int c8 = tid % LPR, rr = tid / LPR;
  const __amdgpu_buffer_rsrc_t rs = rows_rsrc<D>(src, stride, tok0, n, 64);
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) w[ps] = load16(rs, (uint32_t)(((rr + ps * RPP) * stride + c8 * 8) * 2));
}

// The producer's inputs for the rows of one head: the norm weights and the
// rotation rows from `row0` (the flattened (batch, token) index of token 0).
struct ProdRows {
  const ProdArgs* prod;
  const float* nw;
  int64_t row0;
};

// Q, or K without smoothing (mu == nullptr), or K smoothed by the head's bf16
// mean mu[D] (in LDS): codes in row-fragment order and scales of one 64-token
// block from the loads of rows_load.  PROD: rows of the projection output
// through RMSNorm + rotary (pr: the block's weights and rotations).  TAIL: the
// block reaches past N.
template <int D, int QK, int GRAN, bool PROD, bool TAIL>
__device__ __forceinline__ void rows_quant(uint4 (&w)[64 / (256 / (D / 8))], const ProdRows& pr,
                                           int64_t tok0, int64_t n, float fold,
                                           const float* mu, uint8_t* __restrict__ codes, float* __restrict__ scale,
                                           unsigned* blk_amax, int tid) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  const int c8 = tid % LPR, rr = tid / LPR;
  if constexpr (PROD) {
    const float r = tokens_rrms<D, PASSES>(w, pr.prod->eps, tid);
    float wn[8];
    load_w8(pr.nw, c8, wn);
#pragma unroll
    for (int ps = 0; ps < PASSES; ++ps) {
      f32x4 fr[4];
      load_freqs<D>(pr.prod->freqs, pr.row0 + min(tok0 + rr + ps * RPP, n - 1), c8, fr);
      w[ps] = rope8(w[ps], quad_lane(r, ps), wn, fr);
      if (tok0 + rr + ps * RPP >= n) w[ps] = make_uint4(0, 0, 0, 0);  // +0 codes past N
    }
  }
  float x[PASSES][8], amax[PASSES];
  float m[8];
  if (mu != nullptr) {
    const f32x4* m4 = reinterpret_cast<const f32x4*>(mu + c8 * 8);
    const f32x4 a = m4[0], b = m4[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m[i] = a[i];
      m[4 + i] = b[i];
    }
  }
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    unpack8(w[ps], x[ps]);
    if (mu != nullptr) {
      // bf16(k - mean); rows past N (loaded as zeros) stay zero
      const float keep = (!TAIL || tok0 + rr + ps * RPP < n) ? 1.0f : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t p2 = pack_bf16x2(x[ps][e] - m[e], x[ps][e + 1] - m[e + 1]);  // round to nearest even
        x[ps][e] = __uint_as_float(p2 << 16);
        x[ps][e + 1] = __uint_as_float(p2 & 0xffff0000u);
        if constexpr (TAIL) {
          x[ps][e] *= keep;
          x[ps][e + 1] *= keep;
        }
      }
    }
  }
  row_amax<D, GRAN, PASSES>(x, amax, blk_amax);
  store_rows<D, QK, GRAN, PASSES>(x, amax, tok0, rr, c8, fold, codes, scale, tid);
}

template <int D, int QK, int GRAN, bool PROD>
__device__ __forceinline__ void rows_block(const uint16_t* src, int64_t stride, int64_t row0, const float* nw,
                                           const ProdArgs& prod, int64_t tok0, int64_t n, float fold,
                                           uint8_t* __restrict__ codes, float* __restrict__ scale, unsigned* blk_amax,
                                           int tid) {
  uint4 w[64 / (256 / (D / 8))];
  rows_load<D>(src, stride, tok0, n, tid, w);
  rows_quant<D, QK, GRAN, PROD, false>(w, ProdRows{&prod, nw, row0}, tok0, n, fold, nullptr, codes, scale, blk_amax,
                                       tid);
}

// V of one 64-token block: per-channel fp8 scales and codes, or bf16, in the
// P.V operand's fragment order.  Lane (g, c8) holds channels [8*c8, +8) of the
// 4 consecutive tokens 4g..4g+3, so the 4 codes of a channel form one 32-bit
// fragment word.  The image is assembled in LDS and written as contiguous
// 16-byte chunks.
template <int D, int PV>
__device__ __forceinline__ void v_block(const uint16_t* src, int64_t stride, int64_t tok0, int64_t n, int64_t blk,
                                        int bh, int64_t np, uint8_t* __restrict__ vout, float* __restrict__ vs,
                                        uint8_t* lds, int tid) {
  constexpr int LPR = D / 8;
  constexpr int VTHREADS = 16 * LPR;  // 16 groups of 4 tokens
  constexpr int VW = VTHREADS / 64;   // waves holding V
  using L = QuantLds<D, PV>;
  float* vmax = reinterpret_cast<float*>(lds + L::kVmax);
  float* vinv = reinterpret_cast<float*>(lds + L::kInv);
  uint8_t* vimg = lds + L::kImg;
  const int wave = tid >> 6, c8 = tid % LPR;
  const int g = (tid / LPR) & 15;
  const __amdgpu_buffer_rsrc_t rs = rows_rsrc<D>(src, stride, tok0, n, 64);
  uint4 vw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    vw[i] = tid < VTHREADS ? load16(rs, (uint32_t)(((4 * g + i) * stride + c8 * 8) * 2)) : make_uint4(0, 0, 0, 0);
  const int64_t co = (int64_t)bh * np * D;
  if constexpr (PV == kPV_FP8) {
    // channel maxima of |v| over the 4 tokens, on the bf16 bit patterns (for
    // non-NaN values the magnitude bits order like the magnitudes)
    float cm[8];
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      u16x2 mm = __builtin_bit_cast(u16x2, word_of(vw[0], w4) & 0x7fff7fffu);
#pragma unroll
      for (int i = 1; i < 4; ++i) mm = __builtin_elementwise_max(mm, __builtin_bit_cast(u16x2, word_of(vw[i], w4) & 0x7fff7fffu));
      cm[2 * w4] = __uint_as_float((uint32_t)mm.x << 16);
      cm[2 * w4 + 1] = __uint_as_float((uint32_t)mm.y << 16);
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
      f32x4* o4 = reinterpret_cast<f32x4*>(vmax + wave * D + c8 * 8);
      o4[0] = f32x4{cm[0], cm[1], cm[2], cm[3]};
      o4[1] = f32x4{cm[4], cm[5], cm[6], cm[7]};
    }
    __syncthreads();
    // one thread per channel: the block's maximum, its scale and inverse
    if (tid < D) {
      float am = vmax[tid];
#pragma unroll
      for (int ww = 1; ww < VW; ++ww) am = fmaxf(am, vmax[ww * D + tid]);
      vinv[tid] = kFp8Max / fmaxf(am, kEps);
      vs[((int64_t)bh * (np / 64) + blk) * D + tid] = am / kFp8Max;
    }
    __syncthreads();
    if (tid < VTHREADS) {
      float inv[8];
      {
        const f32x4* i4 = reinterpret_cast<const f32x4*>(vinv + c8 * 8);
        const f32x4 a = i4[0], b = i4[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          inv[i] = a[i];
          inv[4 + i] = b[i];
        }
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
  constexpr int VBYTES = (PV == kPV_FP8 ? 1 : 2) * 64 * D;
  uint8_t* vo = vout + (PV == kPV_FP8 ? 1 : 2) * (co + tok0 * D);
#pragma unroll
  for (int i = tid; i < VBYTES / 16; i += 256)
    reinterpret_cast<uint4*>(vo)[i] = reinterpret_cast<const uint4*>(vimg)[i];
}

// fp64 column sums of K over one chunk (k_sum_tokens tokens) of one head.
// Lane (rr, c8) holds channels [8*c8, +8) of tokens rr + RPP*ps; the lanes of
// a column are added in a fixed tree, then the 4 waves through ksw (LDS,
// 4 * D doubles).  Returns the chunk's sum of column tid for tid < D (after a
// workgroup barrier; callers synchronize again before reusing ksw).  Every
// sum is formed in a fixed order, so the result does not depend on
// scheduling or on which workgroup computes it.
template <int D, bool PROD, int GROUP = (PROD ? 4 : 8)>
__device__ __forceinline__ double chunk_colsum(const uint16_t* src, int64_t stride, int64_t row0, const ProdArgs& prod,
                                               int64_t ch, int64_t n, double* ksw, int tid) {
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  // GROUP: tokens per lane loaded together
  const int wave = tid >> 6, c8 = tid % LPR, rr = tid / LPR;
  const int64_t ct = k_sum_tokens(n, D);
  const int64_t tok0 = ch * ct;
  float kn[8];
  if constexpr (PROD) load_w8(prod.kw, c8, kn);
  double cs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) cs[e] = 0.0;
  // 256-token pieces (one buffer resource each: 32-bit offsets), GROUP rows per lane at a time
#pragma unroll 1
  for (int64_t t0 = tok0; t0 < min(tok0 + ct, n); t0 += 256) {
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc<D>(src, stride, t0, n, 256);
#pragma unroll 1
    for (int g0 = 0; g0 < 256 / RPP; g0 += GROUP) {
      uint4 w[GROUP];
#pragma unroll
      for (int i = 0; i < GROUP; ++i) w[i] = load16(rs, (uint32_t)(((rr + (g0 + i) * RPP) * stride + c8 * 8) * 2));
      if constexpr (PROD) {
        const float r = tokens_rrms<D, GROUP>(w, prod.eps, tid);
#pragma unroll
        for (int i = 0; i < GROUP; ++i) {
          f32x4 fr[4];
          load_freqs<D>(prod.freqs, row0 + min(t0 + rr + (g0 + i) * RPP, n - 1), c8, fr);
          w[i] = rope8(w[i], quad_lane(r, i), kn, fr);  // zero rows stay zero
        }
      }
#pragma unroll
      for (int i = 0; i < GROUP; ++i) {
        float x[8];
        unpack8(w[i], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) cs[e] += (double)x[e];
      }
    }
  }
  // token rows of the wave (lanes c8 + LPR*m), then the 4 waves
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) cs[e] += __shfl_xor(cs[e], off);
  if ((tid & 63) < LPR) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ksw[wave * D + c8 * 8 + e] = cs[e];
  }
  __syncthreads();
  return tid < D ? (ksw[tid] + ksw[D + tid]) + (ksw[2 * D + tid] + ksw[3 * D + tid]) : 0.0;
}

// The head mean of the smoothing, mu[D] in LDS (fp32 of the bf16 mean), from
// the head's chunk sums: thread j = tid / D of column tid % D adds chunks j,
// j + TPC, ... in order (mt: its kMeanLoads loaded sums, zero past nch), then
// the TPC partial sums of a column are added in order; / N in fp64, rounded
// to fp32 then bf16 (the reference's bf16 mean).  kmean: written when not null.
template <int D>
__device__ __forceinline__ void head_mean(double s, int64_t n, double (*msum)[D], float* mu, uint16_t* kmean,
                                          int tid) {
  constexpr int TPC = 256 / D;
  msum[tid / D][tid % D] = s;
  __syncthreads();
  if (tid < D) {
    double t = msum[0][tid];
#pragma unroll
    for (int j = 1; j < TPC; ++j) t += msum[j][tid];
    const uint16_t m16 = f32_to_bf16_rne((float)(t / (double)n));
    mu[tid] = bf16_to_f32(m16);
    if (kmean != nullptr) kmean[tid] = m16;
  }
  __syncthreads();
}

// Loads of the head's chunk sums for head_mean (clamped in bounds so they
// issue without branches; values past nch are dropped by mean_sum).
template <int D, bool COHERENT = false>
__device__ __forceinline__ void load_chunk_sums(const double* hp, int64_t nch, int tid, double (&mt)[kMeanLoads]) {
  constexpr int TPC = 256 / D;
#pragma unroll
  for (int i = 0; i < kMeanLoads; ++i) {
    const double* p = hp + min((int64_t)(tid / D + TPC * i), nch - 1) * D;
    if constexpr (COHERENT)
      mt[i] = __builtin_bit_cast(double, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT));
    else
      mt[i] = *p;
  }
}
template <int D>
__device__ __forceinline__ double mean_sum(const double (&mt)[kMeanLoads], int64_t nch, int tid) {
  constexpr int TPC = 256 / D;
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kMeanLoads; ++i) s += tid / D + TPC * i < nch ? mt[i] : 0.0;
  return s;
}

// First quantization kernel of the two-kernel form: one role per workgroup,
// 1D grid with every role of every head of the same rows adjacent.
//   SMOOTH: units [0, nch * BH) the K column sums of chunk u / BH of head
//           u % BH; then unit 2 * (blk * BH + head) + role, role 0 = Q, 1 = V.
//   else:   unit 3 * (blk * BH + head) + role, role 2 = K.
// The longest workgroups (column sums) are dispatched first, and the short
// block roles fill the CUs around them.
template <int D, int QK, int PV, int GRAN, bool SMOOTH, bool PROD>
__global__ void __launch_bounds__(256) quantize_qv_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t bhn,
    int64_t n, int64_t np, float fold, double* __restrict__ ksum_part, uint8_t* __restrict__ qc,
    float* __restrict__ qs, uint8_t* __restrict__ kc, float* __restrict__ ks, uint8_t* __restrict__ vout,
    float* __restrict__ vs, ProdArgs prod) {
  using L = QuantLds<D, PV>;
  constexpr int ROLES = SMOOTH ? 2 : 3;
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::kTotal];
  unsigned* blk_amax = reinterpret_cast<unsigned*>(lds + L::kAmax);
  const int tid = threadIdx.x;
  int64_t u = blockIdx.x;
  if constexpr (SMOOTH) {
    const int64_t nch = k_sum_chunks(n, D), nsum = nch * bhn;
    if (u < nsum) {
      const int64_t ch = u / bhn;
      const int bh = (int)(u - ch * bhn);
      const HeadRows<D, PROD> src(q, k, v, prod, bh, n);
      const double cs = chunk_colsum<D, PROD>(src.k, src.stride, src.row0, prod, ch, n,
                                              reinterpret_cast<double*>(lds), tid);
      if (tid < D) ksum_part[((int64_t)bh * nch + ch) * D + tid] = cs;
      return;
    }
    u -= nsum;
  }
  const int role = (int)(u % ROLES);
  const int64_t rest = u / ROLES;
  const int64_t blk = rest / bhn;
  const int bh = (int)(rest - blk * bhn);
  const HeadRows<D, PROD> src(q, k, v, prod, bh, n);
  const int64_t tok0 = blk * 64;
  const int64_t co = (int64_t)bh * np * D;
  const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);
  if (role == 1) {
    v_block<D, PV>(src.v, src.stride, tok0, n, blk, bh, np, vout, vs, lds, tid);
    return;
  }
  if (GRAN == kGRAN_BLOCK64) {
    if (tid == 0) *blk_amax = 0u;
    __syncthreads();
  }
  if (role == 0)
    rows_block<D, QK, GRAN, PROD>(src.q, src.stride, src.row0, prod.qw, prod, tok0, n, fold, qc + co, qs + sco,
                                  blk_amax, tid);
  else
    rows_block<D, QK, GRAN, PROD>(src.k, src.stride, src.row0, prod.kw, prod, tok0, n, 1.0f, kc + co, ks + sco,
                                  blk_amax, tid);
}

// Second quantization kernel of the two-kernel form (smoothing): K of two
// 64-token blocks of one head (the padded length is a multiple of 128),
// shifted by the head's mean; 1D grid, unit y * BH + head.  The chunk sums
// are loaded first (needed first), then the K rows.
template <int D, int QK, int GRAN, bool PROD>
__global__ void __launch_bounds__(256) quantize_k_kernel(const uint16_t* __restrict__ k, int64_t bhn, int64_t n,
                                                         int64_t np, const double* __restrict__ ksum_part,
                                                         uint8_t* __restrict__ kc, float* __restrict__ ks,
                                                         uint16_t* __restrict__ kmean, ProdArgs prod) {
  constexpr int TPC = 256 / D;
  constexpr int PASSES = 64 / (256 / (D / 8));
  __shared__ double msum[TPC][D];
  __shared__ __attribute__((aligned(16))) float mu[D];
  __shared__ unsigned blk_amax[2];
  const int tid = threadIdx.x;
  const int64_t y = blockIdx.x / bhn;
  const int bh = (int)(blockIdx.x - y * bhn);
  const int64_t tok0 = y * 128;
  const HeadRows<D, PROD> src(k, k, k, prod, bh, n);
  const int64_t nch = k_sum_chunks(n, D);  // at most kMeanLoads * TPC
  double mt[kMeanLoads];
  load_chunk_sums<D>(ksum_part + (int64_t)bh * nch * D + tid % D, nch, tid, mt);
  uint4 w0[PASSES], w1[PASSES];
  rows_load<D>(src.k, src.stride, tok0, n, tid, w0);
  rows_load<D>(src.k, src.stride, tok0 + 64, n, tid, w1);
  if (GRAN == kGRAN_BLOCK64 && tid < 2) blk_amax[tid] = 0u;
  head_mean<D>(mean_sum<D>(mt, nch, tid), n, msum, mu, y == 0 ? kmean + (int64_t)bh * D : nullptr, tid);
  const int64_t co = (int64_t)bh * np * D;
  const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);
  const ProdRows pr{&prod, prod.kw, src.row0};
  if (tok0 + 128 <= n) {
    rows_quant<D, QK, GRAN, PROD, false>(w0, pr, tok0, n, 1.0f, mu, kc + co, ks + sco, &blk_amax[0], tid);
    rows_quant<D, QK, GRAN, PROD, false>(w1, pr, tok0 + 64, n, 1.0f, mu, kc + co, ks + sco, &blk_amax[1], tid);
  } else {
    rows_quant<D, QK, GRAN, PROD, true>(w0, pr, tok0, n, 1.0f, mu, kc + co, ks + sco, &blk_amax[0], tid);
    rows_quant<D, QK, GRAN, PROD, true>(w1, pr, tok0 + 64, n, 1.0f, mu, kc + co, ks + sco, &blk_amax[1], tid);
  }
}

// Waits until every chunk flag of head bh shows this call's epoch, for at most
// spin_limit rounds of s_sleep; returns whether they all did (uniform).
__device__ __forceinline__ bool wait_head_flags(const uint64_t* __restrict__ hf, int64_t nch, uint64_t epoch,
                                                int spin_limit, int tid) {
  uint64_t f = tid < nch ? __hip_atomic_load(&hf[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
  bool ready = __syncthreads_and(f == epoch);
  for (int r = 0; !ready && r < spin_limit; ++r) {
    __builtin_amdgcn_s_sleep(32);
    f = tid < nch ? __hip_atomic_load(&hf[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
    ready = __syncthreads_and(f == epoch);
  }
  return ready;
}

// Thread tid's partial sum of the head mean (for head_mean): from the
// published chunk sums (read with agent-scope relaxed atomic loads, the
// coherence point) when ready, else from the head's chunk sums formed here
// with the same arithmetic and order (chunk_colsum; LDS from lds).
template <int D, bool PROD>
__device__ __forceinline__ double head_sum_part(bool ready, const HeadRows<D, PROD>& src, const ProdArgs& prod,
                                                int bh, int64_t n, int64_t nch, const double* __restrict__ ksum_part,
                                                uint8_t* lds, int tid) {
  constexpr int TPC = 256 / D;
  double s = 0.0;
  if (ready) {
    double mt[kMeanLoads];
    load_chunk_sums<D, true>(ksum_part + (int64_t)bh * nch * D + tid % D, nch, tid, mt);
    s = mean_sum<D>(mt, nch, tid);
  } else {
    double(*msum)[D] = reinterpret_cast<double(*)[D]>(lds);
    double* ksw = reinterpret_cast<double*>(lds + TPC * D * 8 + D * 4);
#pragma unroll 1
    for (int64_t c = 0; c < nch; ++c) {
      const double cs = chunk_colsum<D, PROD, 2>(src.k, src.stride, src.row0, prod, c, n, ksw, tid);
      if (tid < D) msum[0][tid] = cs;  // chunk c's column sums
      __syncthreads();
      if (c % TPC == tid / D) s += msum[0][tid % D];
      __syncthreads();
    }
  }
  return s;
}

// Waves per SIMD the producer form of quantize_one_kernel is compiled for: its
// column-sum, slab and fallback paths would take ~117 VGPRs (4 waves) left to
// themselves; at 5 (at most 102) the compiler reorders instead of spilling,
// and the kernel runs in 51.5 instead of 58 us at 1x4416x30x128 (6 waves:
// spills, slower).
constexpr int kProdWaves = 5;

// Slab units of the producer form with per-token scales: a Q or K unit takes
// the RPP tokens of one pass (lane (rr, c8): token s0 + rr, channels
// [8*c8, +8)) for heads [h0, h1) of batch b.  The lane loads its token's
// rotations once (12 floats) and applies them to every head; the heads go four
// at a time, the four taking the places of the four tokens of rows_quant: one
// reduce-scattered RMS (tokens_rrms) and one quantization division per quad
// serve the four.  K rows are shifted by their head's mean (mu: row h - h0 of
// D floats); codes, scales and zeros past N are those of rows_quant.
template <int D, int QK, bool K>
__device__ __forceinline__ void slab_heads(const ProdArgs& prod, int b, int h0, int h1, int64_t s0, int64_t n,
                                           int64_t np, float fold, const float* mu, uint8_t* __restrict__ codes,
                                           float* __restrict__ scale, int tid) {
#pragma clang fp contract(off)
  constexpr int LPR = D / 8;
  const int c8 = tid % LPR, rr = tid / LPR;
  const int64_t t = s0 + rr;
  const bool valid = t < n;
  const int64_t tc = valid ? t : n - 1;  // clamped: the lanes of a token reduce together
  f32x4 fr[4];
  load_freqs<D>(prod.freqs, (int64_t)b * n + tc, c8, fr);
  float wn[8];
  load_w8(K ? prod.kw : prod.qw, c8, wn);
  const uint16_t* row = prod.qkv + ((int64_t)b * n + tc) * (3LL * prod.h * D) + (K ? (int64_t)prod.h * D : 0) + c8 * 8;
  const float qmax = (QK == kQK_INT8) ? kInt8Max : kFp8Max;
  const int d0 = c8 * 8;
  const int64_t frag = row_frag_offset(t, d0 / 32, (d0 / 16) & 1, D) + (d0 & 8);
#pragma unroll
  for (int it = 0; it < kSlabHeads / 4; ++it) {
    const int hb = h0 + 4 * it;
    if (hb >= h1) break;  // uniform
    uint4 w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const uint4*>(row + (int64_t)min(hb + j, h1 - 1) * D);
    const float r = tokens_rrms<D, 4>(w, prod.eps, tid);
    float x[4][8], amax[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 y = valid ? rope8(w[j], quad_lane(r, j), wn, fr) : make_uint4(0, 0, 0, 0);
      unpack8(y, x[j]);
      if constexpr (K) {
        // bf16(k - mean); rows past N stay zero
        const f32x4* m4 = reinterpret_cast<const f32x4*>(mu + (min(hb + j, h1 - 1) - h0) * D + d0);
        const f32x4 ma = m4[0], mb = m4[1];
        const float m[8] = {ma[0], ma[1], ma[2], ma[3], mb[0], mb[1], mb[2], mb[3]};
        const float keep = valid ? 1.0f : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const uint32_t p2 = pack_bf16x2(x[j][e] - m[e], x[j][e + 1] - m[e + 1]);  // round to nearest even
          x[j][e] = __uint_as_float(p2 << 16) * keep;
          x[j][e + 1] = __uint_as_float(p2 & 0xffff0000u) * keep;
        }
      }
    }
    row_amax<D, kGRAN_TOKEN, 4>(x, amax, nullptr);
    // the division of head c8 % 4 in each lane, handed round the quad (store_rows)
    const int mine = c8 & 3;
    uint32_t amb = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) amb |= __float_as_uint(amax[j]) & (0u - (uint32_t)(mine == j));
    const float am = __uint_as_float(amb);
    const float inv_mine = qmax / fmaxf(am, kEps);  // IEEE division (correctly rounded)
    const float scale_mine = (am / qmax) * fold;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float inv = quad_lane(inv_mine, j);
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = x[j][e] * inv;
      uint2 word;
      if (QK == kQK_INT8) {
        word.x = pack_i8x4(y[0], y[1], y[2], y[3]);
        word.y = pack_i8x4(y[4], y[5], y[6], y[7]);
      } else {
        word.x = pack_fp8x4(y[0], y[1], y[2], y[3]);
        word.y = pack_fp8x4(y[4], y[5], y[6], y[7]);
      }
      if (hb + j < h1) {
        const int64_t bh = (int64_t)b * prod.h + hb + j;
        *reinterpret_cast<uint2*>(codes + bh * np * D + frag) = word;
        if (c8 == j) scale[bh * np + t] = scale_mine;
      }
    }
  }
}

// LDS of a K slab unit (byte offsets): the group's means float [kSlabHeads][D],
// then head_mean's double [TPC][D] and chunk_colsum's double [4][D] for the
// bounded-wait fallback.
template <int D>
struct SlabLds {
  static constexpr int kMu = 0;
  static constexpr int kMsum = kSlabHeads * D * 4;
  static constexpr int kKsw = kMsum + (256 / D) * D * 8;
  static constexpr int kTotal = kKsw + 4 * D * 8;
};

// One-kernel form with smoothing (not used under stream capture: the epoch is
// a launch argument).  1D grid, units in dispatch order:
//   [0, nsum)   K column sums of chunk u / BH of head u % BH; each publishes
//               flag[head][chunk] = epoch after its sums;
//   then rows   the Q, V and K roles of the 64-token blocks, with the K block
//               of row r - lag beside the Q and V blocks of row r (rows
//               0..lag-1 carry only Q and V, the last lag rows only K): the
//               column sums run well ahead of the first K block, and the K
//               blocks overlap the Q/V stream instead of forming a tail.
// Each K workgroup reads its head's flags and proceeds when every chunk shows
// this call's epoch (a 64-bit value the host never reuses, so memory left by
// earlier calls never matches).  The wait is bounded: after spin_limit rounds
// the workgroup forms the chunk sums itself, with the same arithmetic and
// order (chunk_colsum), so every workgroup exits and the codes are the same
// either way.
// With the producer and per-token scales (SLAB) the Q and K roles are slab
// units (slab_heads: one pass of RPP tokens for kSlabHeads heads) and the head means
// are formed once: a column-sum unit that, after its own flag, finds every
// chunk flag of its head set forms the mean (head_mean, the same sums in the
// same order), stores it as fp32 [BH][D] beside the flags and publishes
// mflag[head] = epoch.  Two units may both find it so and store the same
// values; at least one does, because each reads the flags only after its own
// flag store has completed.  Per row: the Q slab units of the block's passes
// (pass-major, hg-head groups within), the block's V units, the K slab units
// of block r - lag.  A K slab unit waits for its heads' mean flags (bounded,
// with the chunk-sum fallback).
template <int D, int QK, int PV, int GRAN, bool PROD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PROD ? kProdWaves : 1))) quantize_one_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t bhn,
    int64_t n, int64_t np, float fold, double* __restrict__ ksum_part, uint64_t* __restrict__ flags,
    uint64_t epoch, int spin_limit, int64_t lag, uint8_t* __restrict__ qc, float* __restrict__ qs,
    uint8_t* __restrict__ kc, float* __restrict__ ks, uint8_t* __restrict__ vout, float* __restrict__ vs,
    uint16_t* __restrict__ kmean, ProdArgs prod) {
  using L = QuantLds<D, PV>;
  constexpr bool SLAB = PROD && GRAN == kGRAN_TOKEN;
  constexpr int TPC = 256 / D;
  constexpr int PASSES = 64 / (256 / (D / 8));
  constexpr int RPP = 256 / (D / 8);
  static_assert(TPC * D * 8 + D * 4 + 4 * D * 8 <= L::kBytes, "K role scratch fits");
  constexpr int kLdsBytes = (SLAB && SlabLds<D>::kTotal > L::kTotal) ? SlabLds<D>::kTotal : L::kTotal;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  unsigned* blk_amax = reinterpret_cast<unsigned*>(lds + L::kAmax);
  const int tid = threadIdx.x;
  const int64_t nch = k_sum_chunks(n, D), nsum = nch * bhn;
  const int64_t nblk = np / 64;
  uint64_t* mflags = flags + bhn * nch;                       // SLAB: [BH] mean flags
  float* kmu = reinterpret_cast<float*>(mflags + bhn);        // SLAB: [BH][D] fp32 means
  int64_t u = blockIdx.x;
  if (u < nsum) {
    const int64_t ch = u / bhn;
    const int bh = (int)(u - ch * bhn);
    const HeadRows<D, PROD> src(q, k, v, prod, bh, n);
    const double cs = chunk_colsum<D, PROD>(src.k, src.stride, src.row0, prod, ch, n,
                                            reinterpret_cast<double*>(lds), tid);
    // The sums and the flag go out as agent-scope relaxed atomic stores, which
    // gfx950 writes through to the device's coherence point (sc1); waiting for
    // the sums' completion before the flag store orders them without the
    // whole-L2 write-back of a release fence.
    if (tid < D)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(ksum_part) + ((int64_t)bh * nch + ch) * D + tid,
                         __builtin_bit_cast(uint64_t, cs), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_vmem();
    __syncthreads();
    if (tid == 0) __hip_atomic_store(&flags[(int64_t)bh * nch + ch], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (SLAB) {
      wait_vmem();  // this unit's flag is at the coherence point before the others are read
      __syncthreads();
      const uint64_t* hf = flags + (int64_t)bh * nch;
      const uint64_t f = tid < nch ? __hip_atomic_load(&hf[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
      if (__syncthreads_and(f == epoch)) {
        double mt[kMeanLoads];
        load_chunk_sums<D, true>(ksum_part + (int64_t)bh * nch * D + tid % D, nch, tid, mt);
        float* mu = reinterpret_cast<float*>(lds + TPC * D * 8);
        head_mean<D>(mean_sum<D>(mt, nch, tid), n, reinterpret_cast<double(*)[D]>(lds), mu,
                     kmean + (int64_t)bh * D, tid);
        if (tid < D)
          __hip_atomic_store(reinterpret_cast<uint32_t*>(kmu) + (int64_t)bh * D + tid, __float_as_uint(mu[tid]),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_vmem();
        __syncthreads();
        if (tid == 0) __hip_atomic_store(&mflags[bh], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;
  }
  u -= nsum;
  if constexpr (SLAB) {
    // head groups: kSlabHeads consecutive heads of one batch, the last fewer
    const int64_t ngb = (prod.h + kSlabHeads - 1) / kSlabHeads, ng = (bhn / prod.h) * ngb;
    const int64_t per = PASSES * ng, per_qv = per + bhn;
    const int64_t seg1 = per_qv * lag, seg2 = (per_qv + per) * (nblk - lag);
    int64_t r, x;  // row, unit within the row
    bool kunit = false;
    if (u < seg1) {
      r = u / per_qv;
      x = u - r * per_qv;
    } else if (u < seg1 + seg2) {
      const int64_t w = u - seg1;
      r = lag + w / (per_qv + per);
      x = w % (per_qv + per);
      if (x >= per_qv) {
        kunit = true;
        x -= per_qv;
        r -= lag;
      }
    } else {
      const int64_t w = u - seg1 - seg2;
      r = nblk - lag + w / per;
      x = w % per;
      kunit = true;
    }
    if (!kunit && x >= per) {  // V of block r, one head
      const int bh = (int)(x - per);
      const HeadRows<D, PROD> src(q, k, v, prod, bh, n);
      v_block<D, PV>(src.v, src.stride, r * 64, n, r, bh, np, vout, vs, lds, tid);
      return;
    }
    const int64_t s0 = r * 64 + (x / ng) * RPP;  // the pass's first token
    const int64_t g = x % ng;
    const int b = (int)(g / ngb), h0 = (int)(g % ngb) * kSlabHeads;
    const int h1 = min(h0 + kSlabHeads, prod.h);
    if (!kunit) {
      slab_heads<D, QK, false>(prod, b, h0, h1, s0, n, np, fold, nullptr, qc, qs, tid);
      return;
    }
    using S = SlabLds<D>;
    float* mug = reinterpret_cast<float*>(lds + S::kMu);
    double(*msum)[D] = reinterpret_cast<double(*)[D]>(lds + S::kMsum);
    double* ksw = reinterpret_cast<double*>(lds + S::kKsw);
    // the group's means, published by the column-sum units: one bounded wait
    // for all their flags, then the rows; a head whose flag is still missing
    // has its mean formed here from its chunk sums
    const int cnt = h1 - h0;
    const int64_t bh0 = (int64_t)b * prod.h + h0;
    const uint32_t* kmu32 = reinterpret_cast<const uint32_t*>(kmu) + bh0 * D;
    uint64_t f = tid < cnt ? __hip_atomic_load(&mflags[bh0 + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
    bool ready = __syncthreads_and(f == epoch);
    for (int it = 0; !ready && it < spin_limit; ++it) {
      __builtin_amdgcn_s_sleep(32);
      f = tid < cnt ? __hip_atomic_load(&mflags[bh0 + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
      ready = __syncthreads_and(f == epoch);
    }
    if (ready) {
      for (int i = tid; i < cnt * D; i += 256)
        mug[i] = __uint_as_float(__hip_atomic_load(kmu32 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    } else {
#pragma unroll 1
      for (int j = 0; j < cnt; ++j) {
        const uint64_t fj =
            tid == 0 ? __hip_atomic_load(&mflags[bh0 + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
        if (__syncthreads_and(fj == epoch)) {
          if (tid < D)
            mug[j * D + tid] = __uint_as_float(
                __hip_atomic_load(kmu32 + j * D + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          continue;
        }
        // the chunk sums of this head, formed here in the same order
        const HeadRows<D, PROD> src(q, k, v, prod, (int)(bh0 + j), n);
        double sj = 0.0;
#pragma unroll 1
        for (int64_t c = 0; c < nch; ++c) {
          const double cs = chunk_colsum<D, PROD, 2>(src.k, src.stride, src.row0, prod, c, n, ksw, tid);
          if (tid < D) msum[0][tid] = cs;  // chunk c's column sums
          __syncthreads();
          if (c % TPC == tid / D) sj += msum[0][tid % D];
          __syncthreads();
        }
        head_mean<D>(sj, n, msum, mug + j * D, nullptr, tid);
      }
    }
    __syncthreads();
    slab_heads<D, QK, true>(prod, b, h0, h1, s0, n, np, 1.0f, mug, kc, ks, tid);
    return;
  } else {
    (void)mflags;
    (void)kmu;
    // block roles with the K blocks `lag` rows behind the Q and V blocks
    int role;
    int64_t blk;
    int bh;
    const int64_t seg1 = 2 * bhn * lag, seg2 = 3 * bhn * (nblk - lag);
    if (u < seg1) {
      role = (int)(u & 1);
      const int64_t rest = u >> 1;
      blk = rest / bhn;
      bh = (int)(rest - blk * bhn);
    } else if (u < seg1 + seg2) {
      const int64_t w = u - seg1;
      role = (int)(w % 3);
      const int64_t rest = w / 3;
      const int64_t r = lag + rest / bhn;
      bh = (int)(rest % bhn);
      blk = role == 2 ? r - lag : r;
    } else {
      const int64_t w = u - seg1 - seg2;
      role = 2;
      blk = nblk - lag + w / bhn;
      bh = (int)(w % bhn);
    }
    if (role != 2) {
      const HeadRows<D, PROD> src(q, k, v, prod, bh, n);
      const int64_t tok0 = blk * 64;
      if (role == 1) {
        v_block<D, PV>(src.v, src.stride, tok0, n, blk, bh, np, vout, vs, lds, tid);
        return;
      }
      if (GRAN == kGRAN_BLOCK64) {
        if (tid == 0) *blk_amax = 0u;
        __syncthreads();
      }
      const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);
      rows_block<D, QK, GRAN, PROD>(src.q, src.stride, src.row0, prod.qw, prod, tok0, n, fold,
                                    qc + (int64_t)bh * np * D, qs + sco, blk_amax, tid);
      return;
    }
    // ---- K of one block ----
    double(*msum)[D] = reinterpret_cast<double(*)[D]>(lds);
    float* mu = reinterpret_cast<float*>(lds + TPC * D * 8);
    double* ksw = reinterpret_cast<double*>(lds + TPC * D * 8 + D * 4);
    const int64_t tok0 = blk * 64;
    const HeadRows<D, PROD> src(q, k, v, prod, bh, n);
    const uint64_t* hf = flags + (int64_t)bh * nch;
    // flags and sums are read with agent-scope relaxed atomic loads, which read
    // the coherence point (sc1), issued only after the flags show this epoch
    uint64_t f = tid < nch ? __hip_atomic_load(&hf[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
    if (GRAN == kGRAN_BLOCK64 && tid == 0) *blk_amax = 0u;
    bool ready = __syncthreads_and(f == epoch);
    for (int r = 0; !ready && r < spin_limit; ++r) {
      __builtin_amdgcn_s_sleep(32);
      f = tid < nch ? __hip_atomic_load(&hf[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : epoch;
      ready = __syncthreads_and(f == epoch);
    }
    double s = 0.0;
    if (ready) {
      double mt[kMeanLoads];
      load_chunk_sums<D, true>(ksum_part + (int64_t)bh * nch * D + tid % D, nch, tid, mt);
      s = mean_sum<D>(mt, nch, tid);
    } else {
      // the chunk sums of this head, formed here in the same order
  #pragma unroll 1
      for (int64_t c = 0; c < nch; ++c) {
        const double cs = chunk_colsum<D, PROD, 2>(src.k, src.stride, src.row0, prod, c, n, ksw, tid);
        if (tid < D) msum[0][tid] = cs;  // chunk c's column sums
        __syncthreads();
        if (c % TPC == tid / D) s += msum[0][tid % D];
        __syncthreads();
      }
    }
    uint4 w[PASSES];
    rows_load<D>(src.k, src.stride, tok0, n, tid, w);  // after the mean: fewer registers live
    head_mean<D>(s, n, msum, mu, blk == 0 ? kmean + (int64_t)bh * D : nullptr, tid);
    const int64_t co = (int64_t)bh * np * D;
    const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);
    const ProdRows pr{&prod, prod.kw, src.row0};
    if (tok0 + 64 <= n)
      rows_quant<D, QK, GRAN, PROD, false>(w, pr, tok0, n, 1.0f, mu, kc + co, ks + sco, blk_amax, tid);
    else
      rows_quant<D, QK, GRAN, PROD, true>(w, pr, tok0, n, 1.0f, mu, kc + co, ks + sco, blk_amax, tid);
  }
}

// Single-read form with smoothing, for heads whose chunks are 256 tokens
// (k_sum_tokens(n, D) == 256; not used under stream capture, nor with the
// producer, whose K units would hold too many registers; prod is unused).  1D grid, head
// after head: the head's nch K units, then its 2 * nblk Q and V block units.
// A K unit loads its 256 tokens once into registers (four 64-token blocks in
// the lane layout of rows_load), adds their fp64 column sums in chunk_colsum's
// order, publishes them and its chunk flag as the column-sum units of
// quantize_one_kernel do, waits for the head's flags (wait_head_flags; after
// a bounded wait it forms the head's chunk sums itself and loads its tokens
// again), then smooths and quantizes the blocks it holds (those below Np).  K is read once:
// a head's K units are consecutive in dispatch order, so every unit a waiting
// one depends on is dispatched before any later head's work, and the bounded
// wait covers the rest.
template <int D, int QK, int PV, int GRAN>
__global__ void __launch_bounds__(256) quantize_fused_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t bhn,
    int64_t n, int64_t np, float fold, double* __restrict__ ksum_part, uint64_t* __restrict__ flags,
    uint64_t epoch, int spin_limit, uint8_t* __restrict__ qc, float* __restrict__ qs, uint8_t* __restrict__ kc,
    float* __restrict__ ks, uint8_t* __restrict__ vout, float* __restrict__ vs, uint16_t* __restrict__ kmean,
    ProdArgs prod) {
  using L = QuantLds<D, PV>;
  constexpr int LPR = D / 8;
  constexpr int RPP = 256 / LPR;
  constexpr int PASSES = 64 / RPP;
  constexpr int TPC = 256 / D;
  static_assert(TPC * D * 8 + D * 4 + 4 * D * 8 <= L::kBytes, "K role scratch fits");
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::kTotal];
  unsigned* blk_amax = reinterpret_cast<unsigned*>(lds + L::kAmax);
  const int tid = threadIdx.x;
  const int64_t nch = k_sum_chunks(n, D);
  const int64_t nblk = np / 64;
  const int64_t per_head = nch + 2 * nblk;
  const int bh = (int)(blockIdx.x / per_head);
  const int64_t u = blockIdx.x - (int64_t)bh * per_head;
  const HeadRows<D, false> src(q, k, v, prod, bh, n);
  if (u >= nch) {
    const int role = (int)((u - nch) & 1);
    const int64_t blk = (u - nch) >> 1;
    const int64_t tok0 = blk * 64;
    if (role == 1) {
      v_block<D, PV>(src.v, src.stride, tok0, n, blk, bh, np, vout, vs, lds, tid);
      return;
    }
    if (GRAN == kGRAN_BLOCK64) {
      if (tid == 0) *blk_amax = 0u;
      __syncthreads();
    }
    const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);
    rows_block<D, QK, GRAN, false>(src.q, src.stride, src.row0, prod.qw, prod, tok0, n, fold,
                                  qc + (int64_t)bh * np * D, qs + sco, blk_amax, tid);
    return;
  }
  // ---- K of one 256-token chunk, read once ----
  const int64_t ch = u;
  const int64_t tok0 = ch * 256;
  const int wave = tid >> 6, c8 = tid % LPR, rr = tid / LPR;
  uint4 w[4][PASSES];
  // the chunk's 256 tokens
  auto load_chunk = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 4; ++b) rows_load<D>(src.k, src.stride, tok0 + 64 * b, n, tid, w[b]);
  };
  load_chunk();
  if (GRAN == kGRAN_BLOCK64 && tid < 4) blk_amax[tid] = 0u;
  {
    // column sums: each lane adds its tokens rr, rr + RPP, ... in order, then
    // the lanes of a column in a fixed tree, then the 4 waves in order (the
    // order of chunk_colsum)
    double cs[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) cs[e] = 0.0;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int ps = 0; ps < PASSES; ++ps) {
        float x[8];
        unpack8(w[b][ps], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) cs[e] += (double)x[e];
        __builtin_amdgcn_sched_barrier(0);  // one piece at a time: the held blocks stay packed
      }
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) cs[e] += __shfl_xor(cs[e], off);
    double* ksw = reinterpret_cast<double*>(lds + TPC * D * 8 + D * 4);
    if ((tid & 63) < LPR) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ksw[wave * D + c8 * 8 + e] = cs[e];
    }
    __syncthreads();
    const double col = tid < D ? (ksw[tid] + ksw[D + tid]) + (ksw[2 * D + tid] + ksw[3 * D + tid]) : 0.0;
    if (tid < D)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(ksum_part) + ((int64_t)bh * nch + ch) * D + tid,
                         __builtin_bit_cast(uint64_t, col), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_vmem();
    __syncthreads();  // also ends every read of ksw
    if (tid == 0) __hip_atomic_store(&flags[(int64_t)bh * nch + ch], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const bool ready = wait_head_flags(flags + (int64_t)bh * nch, nch, epoch, spin_limit, tid);
  const double s = head_sum_part<D, false>(ready, src, prod, bh, n, nch, ksum_part, lds, tid);
  if (!ready) load_chunk();  // (rare) the tokens again: none stay in registers while the sums are formed
  head_mean<D>(s, n, reinterpret_cast<double(*)[D]>(lds), reinterpret_cast<float*>(lds + TPC * D * 8),
               ch == 0 ? kmean + (int64_t)bh * D : nullptr, tid);
  const float* mu = reinterpret_cast<const float*>(lds + TPC * D * 8);
  const int64_t co = (int64_t)bh * np * D;
  const int64_t sco = (GRAN == kGRAN_TOKEN) ? (int64_t)bh * np : (int64_t)bh * (np / 64);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t t0 = tok0 + 64 * b;
    __builtin_amdgcn_sched_barrier(0);  // one block at a time
    if (t0 >= np) break;  // uniform: blocks past the padded length hold no codes
    if (t0 + 64 <= n)
      rows_quant<D, QK, GRAN, false, false>(w[b], ProdRows{}, t0, n, 1.0f, mu, kc + co, ks + sco, &blk_amax[b], tid);
    else
      rows_quant<D, QK, GRAN, false, true>(w[b], ProdRows{}, t0, n, 1.0f, mu, kc + co, ks + sco, &blk_amax[b], tid);
  }
}

// Quantization launch form: one kernel unless the stream is capturing
// (default: the single-read form for large launches whose heads have
// 256-token chunks, else the lagged form), or forced by SAGE_QUANT_PATH:
// "two" (two kernels), "lagged" (the lagged one-kernel form), "fused" (the
// single-read form wherever it applies), "fallback" (the default one-kernel
// form with K workgroups that skip the wait and form the chunk sums
// themselves; for tests).
enum { kQuantAuto = 0, kQuantTwoKernels = 1, kQuantOneFallback = 2, kQuantLagged = 3, kQuantFused = 4 };
int quant_path() {
  const char* e = std::getenv("SAGE_QUANT_PATH");
  if (e == nullptr) return kQuantAuto;
  if (std::strcmp(e, "two") == 0) return kQuantTwoKernels;
  if (std::strcmp(e, "fallback") == 0) return kQuantOneFallback;
  if (std::strcmp(e, "lagged") == 0) return kQuantLagged;
  if (std::strcmp(e, "fused") == 0) return kQuantFused;
  return kQuantAuto;
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
  int path;  // kQuantAuto, kQuantTwoKernels, kQuantOneFallback, kQuantLagged
};

constexpr int64_t kLagUnits = 2048;  // Q and V head blocks dispatched ahead of the first K workgroup
constexpr int64_t kFusedMinTokens = 1 << 18;  // head tokens (B * H * N) from which the single-read form runs

// A 64-bit value never passed to an earlier launch of this process: a clock
// reading at first use (distinct across processes) plus a call counter.
uint64_t next_epoch() {
  static std::atomic<uint64_t> counter{0};
  static const uint64_t base =
      (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count() * 0x9E3779B97F4A7C15ull;
  return base + counter.fetch_add(1, std::memory_order_relaxed) * 2 + 1;
}

template <int D, int QK, int PV, int GRAN, bool SMOOTH, bool PROD>
hipError_t launch_quantize_t(const QuantCall& a, hipStream_t st) {
  const int64_t np = padded_len(a.n);
  const int64_t nblk = np / 64;
  if constexpr (SMOOTH) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t ce = hipStreamIsCapturing(st, &cap);
    if (ce != hipSuccess) return ce;
    if (a.path != kQuantTwoKernels && cap == hipStreamCaptureStatusNone) {
      const int64_t nch = k_sum_chunks(a.n, D);
      uint64_t* flags = reinterpret_cast<uint64_t*>(a.ws + a.bh * nch * D);
      const int spin = a.path == kQuantOneFallback ? 0 : 4096;
      // the single-read form for launches of at least kFusedMinTokens head
      // tokens (measured: 4 x 30 x 4352 x 128 135.0 -> 118.8 us; at 30 x
      // 4416 its halved occupancy and each K unit's serial wait make it slower,
      // 31.3 -> 37.5 us), when a head's chunks are 256 tokens
      if constexpr (!PROD) {
        const bool fits = k_sum_tokens(a.n, D) == 256;
        const bool big = a.bh * a.n >= kFusedMinTokens;
        if (fits && (a.path == kQuantFused || (a.path != kQuantLagged && big))) {
          const int64_t grid = a.bh * (nch + 2 * nblk);
          hipLaunchKernelGGL((quantize_fused_kernel<D, QK, PV, GRAN>), dim3((unsigned)grid), dim3(256), 0, st,
                             a.q, a.k, a.v, a.bh, a.n, np, a.fold, a.ws, flags, next_epoch(), spin, a.qc, a.qs,
                             a.kc, a.ks, a.vout, a.vs, a.kmean, a.prod);
          return hipGetLastError();
        }
      }
      constexpr bool SLAB = PROD && GRAN == kGRAN_TOKEN;
      constexpr int PASSES = 64 / (256 / (D / 8));
      // slab units: PASSES per block for each group of kSlabHeads heads of a batch
      const int64_t groups = SLAB ? (a.bh / a.prod.h) * ((a.prod.h + kSlabHeads - 1) / kSlabHeads) : 0;
      const int64_t grid = nch * a.bh + nblk * (SLAB ? a.bh + 2 * PASSES * groups : 3 * a.bh);
      const int64_t lag = min(nblk, (kLagUnits + 2 * a.bh - 1) / (2 * a.bh));
      hipLaunchKernelGGL((quantize_one_kernel<D, QK, PV, GRAN, PROD>), dim3((unsigned)grid), dim3(256), 0, st, a.q,
                         a.k, a.v, a.bh, a.n, np, a.fold, a.ws, flags, next_epoch(), spin, lag, a.qc, a.qs, a.kc,
                         a.ks, a.vout, a.vs, a.kmean, a.prod);
      return hipGetLastError();
    }
  }
  constexpr int ROLES = SMOOTH ? 2 : 3;
  const int64_t nsum = SMOOTH ? k_sum_chunks(a.n, D) * a.bh : 0;
  hipLaunchKernelGGL((quantize_qv_kernel<D, QK, PV, GRAN, SMOOTH, PROD>), dim3((unsigned)(nsum + ROLES * nblk * a.bh)),
                     dim3(256), 0, st, a.q, a.k, a.v, a.bh, a.n, np, a.fold, a.ws, a.qc, a.qs, a.kc, a.ks, a.vout,
                     a.vs, a.prod);
  if (SMOOTH) {
    hipLaunchKernelGGL((quantize_k_kernel<D, QK, GRAN, PROD>), dim3((unsigned)(nblk / 2 * a.bh)), dim3(256), 0, st,
                       a.k, a.bh, a.n, np, a.ws, a.kc, a.ks, a.kmean, a.prod);
  }
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
  const QuantCall a{q, k, v, bh, n, fold, ws, qc, qs, kc, ks, vout, vs, kmean, prod, quant_path()};
  if (d == 128) return launch_quantize_d<128>(qk, pv, gran, smooth, a, st);
  if (d == 64) return launch_quantize_d<64>(qk, pv, gran, smooth, a, st);
  return hipErrorInvalidValue;
}

hipError_t launch_qkv_postprocess(const ProdArgs& prod, int64_t bh, int64_t n, int64_t d, uint16_t* q_out,
                                  uint16_t* k_out, uint16_t* v_out, hipStream_t st) {
  const int64_t rpp = 256 / (d / 8);  // tokens per slab
  const int64_t groups = (prod.h + kSlabHeads - 1) / kSlabHeads;
  const dim3 grid((unsigned)((bh / prod.h) * ((n + rpp - 1) / rpp) * groups));
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

// Workgroups of the largest quantization launch: the column-sum chunks plus
// three roles per 64-token block, for every head; with the producer (h > 0
// heads per batch) also the slab form's chunks, V blocks and two slab units
// per pass of a block for each group of kSlabHeads heads.
int64_t quant_grid_units(int64_t bh, int64_t n, int64_t d, int64_t h) {
  const int64_t nch = k_sum_chunks(n, d), nblk = padded_len(n) / 64;
  const int64_t plain = (nch + 3 * nblk) * bh;
  if (h <= 0) return plain;
  const int64_t groups = (bh / h) * ((h + kSlabHeads - 1) / kSlabHeads), passes = d / 32;
  return std::max(plain, nch * bh + nblk * (bh + 2 * passes * groups));
}

// fp64 column sums of K per head and chunk, [bh][nch][d], then the chunks'
// flags of the one-kernel form, uint64 [bh][nch], then (its producer form)
// the heads' mean flags, uint64 [bh], and means, fp32 [bh][d].
size_t quant_workspace_bytes(int64_t bh, int64_t n, int64_t d) {
  const int64_t nch = k_sum_chunks(n, d);
  return (size_t)(bh * nch * d) * sizeof(double) + (size_t)(bh * nch + bh) * sizeof(uint64_t) +
         (size_t)(bh * d) * sizeof(float);
}

}  // namespace sage
