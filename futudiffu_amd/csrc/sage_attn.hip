// Fused Sage attention forward for gfx950 (CDNA4).
//
// Reference: the Triton kernels of sqcu/futudiffu src/futudiffu/sage_kernels.py,
// production variant _sage_attn_fwd_int8qk_bf16pv_masked_lse (:1378-1477),
// fp8-QK variants (:215-315) and the fp8 P/V stage of
// _sage_attn_fwd_fp8qk_fp8pv_lse (:1135-1154).
//
// Work decomposition: one workgroup = 4 waves = 128 query rows (the
// reference's Q tile, so the reference tile mask is workgroup-uniform); each
// wave owns 32 query rows.  Keys stream in 64-key tiles (the reference's KV
// tile) staged through LDS in the fragment order the quantize kernel wrote.
//
// Per wave and tile:
//   S^T[key][query] = K . Q^T with v_mfma_i32_32x32x32_i8 (int8) or
//   v_mfma_f32_32x32x64_f8f6f4 (fp8); lane (h, r) holds query r and keys
//   32b + 8j + 4h + i, so every per-query quantity is lane-local.
//   Online softmax in fp32 with exp2 (log2-domain scores).
//   O[query][d] += P . V with v_mfma_f32_32x32x64_f8f6f4 (fp8 P, fp8 V, one
//   dequant FMA per tile for the per-(64-key block, channel) V scale) or
//   v_mfma_f32_32x32x16_bf16 (bf16 P, bf16 V).  P feeds the MFMA straight from
//   the S^T registers: lane (h, r) already holds the keys its A-operand needs.
//
// P scaling (documented deviation from sage_kernels.py:1137-1141): the
// reference scales P per (row, 64-key block) by its block max.  Here P is
// scaled relative to a per-row reference point m that only moves when a
// tile's row max exceeds it by more than TAU (log2 units): p = 2^(s - m) is
// then <= 2^TAU, quantized as e4m3(p * 448 / 2^TAU), and every tile shares one
// P scale, so the PV accumulator needs no per-tile P dequantization and the
// O rescale runs only on the rare tiles where m moves.
#include "sage_common.h"
#include "sage_launch.h"

namespace sage {

constexpr float kTau = 2.0f;
constexpr float kLog2Fp8Max = 8.807354922057604f;  // log2(448)

// Tile class for one wave: 0 = nothing visible, 1 = everything visible,
// 2 = per-token mask needed.
__device__ __forceinline__ int classify(int4 qsum, int4 ksum) {
  if (qsum.z + qsum.w == 0) return 0;         // no query row below N
  if (ksum.z == 0) return 0;                  // no valid key
  if (qsum.z == 0) return ksum.w == 0 ? 1 : 2;  // only padded queries: they see every valid key
  if (qsum.w == 0 && (qsum.y < ksum.x || ksum.y < qsum.x)) return 0;
  if (ksum.w == 0 && ksum.x == ksum.y && qsum.x == qsum.y && qsum.x == ksum.x) return 1;
  return 2;
}

__global__ void doc_summary_kernel(const int32_t* __restrict__ doc, int64_t n, int64_t np, int nb, int nt,
                                   int4* __restrict__ kv_sum, int4* __restrict__ q_sum) {
  const int64_t nq32 = np / 32;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_b = nt + nq32;
  if (idx >= (int64_t)nb * per_b) return;
  const int b = (int)(idx / per_b);
  const int64_t w = idx % per_b;
  int64_t t0, len;
  int4* dst;
  if (w < nt) {
    t0 = w * 64;
    len = 64;
    dst = kv_sum + (int64_t)b * nt + w;
  } else {
    t0 = (w - nt) * 32;
    len = 32;
    dst = q_sum + (int64_t)b * nq32 + (w - nt);
  }
  int mn = 0x7fffffff, mx = -0x7fffffff, nv = 0, ni = 0;
  for (int64_t i = t0; i < t0 + len && i < n; ++i) {
    const int dd = doc[(int64_t)b * n + i];
    if (dd >= 0) {
      mn = min(mn, dd);
      mx = max(mx, dd);
      ++nv;
    } else {
      ++ni;
    }
  }
  *dst = make_int4(mn, mx, nv, ni);
}

template <int D, int PV>
struct Smem {
  static constexpr int kBytes = 64 * D;                            // K codes
  static constexpr int vBytes = (PV == kPV_FP8 ? 64 : 128) * D;    // V codes / bf16
  static constexpr int offV = kBytes;
  static constexpr int offKd = offV + vBytes;                      // 64 fp32 key scales
  static constexpr int offVd = offKd + 256;                        // D fp32 V scales
  static constexpr int offDoc = offVd + 4 * D;                     // 64 int32 key docs
  static constexpr int offXch = offDoc + 256;                      // 4 waves x 32 fp32
  static constexpr int offFlag = offXch + 512;
  static constexpr int total = offFlag + 16;
};

template <int D, int QK, int PV, int GRAN, int MASK>
__global__ void __launch_bounds__(256, 2) attn_fwd_kernel(AttnParams p) {
  using S = Smem<D, PV>;
  constexpr int NC = D / 32;  // 32-channel chunks
  __shared__ __attribute__((aligned(16))) uint8_t smem[S::total];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, r = lane & 31;
  const int qt = blockIdx.x, bh = blockIdx.y;
  const int bidx = bh / p.h;
  const int64_t q0 = (int64_t)qt * kRowsPerWG + 32 * wave;  // first query row of this wave

  // Q fragments (B operand), resident for the whole key loop.
  i32x4 qf[NC];
  {
    const uint8_t* qb = p.qc + (int64_t)bh * p.np * D + (q0 >> 5) * (32 * D);
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const i32x4*>(qb + (c * 64 + lane) * 16);
  }
  float qd;
  if (GRAN == kGRAN_TOKEN)
    qd = p.qs[(int64_t)bh * p.np + q0 + r];
  else
    qd = p.qs[(int64_t)bh * (p.np / 64) + (q0 >> 6)];

  int dq = 0;
  int4 qsum = make_int4(0, 0, 0, 0);
  if (MASK & 2) {
    const int64_t qq = q0 + r;
    dq = qq < p.n ? p.doc[(int64_t)bidx * p.n + qq] : -1;
    qsum = p.q_sum[(int64_t)bidx * (p.np / 32) + (q0 >> 5)];
  }

  const float c0 = (PV == kPV_FP8) ? (kLog2Fp8Max - kTau) : 0.0f;
  float m_ref = -INFINITY;
  float l_acc = 0.0f;
  f32x16 o[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) o[j] = f32x16{0};

  float* xch = reinterpret_cast<float*>(smem + S::offXch) + 32 * wave;
  int* flags = reinterpret_cast<int*>(smem + S::offFlag);
  const uint8_t* kg = p.kc + (int64_t)bh * p.np * D;
  const uint8_t* vg = p.vin + (int64_t)bh * p.np * D * (PV == kPV_FP8 ? 1 : 2);

  for (int t = 0; t < p.nt; ++t) {
    // ---- decide what this wave / workgroup does with tile t ----------------
    int cls = 1;
    if (MASK & 1) {
      if (p.tile_mask[(int64_t)bh * p.mask_stride_z + (int64_t)qt * p.mask_nkv + t] == 0) cls = 0;
    }
    if ((MASK & 2) && cls) cls = classify(qsum, p.kv_sum[(int64_t)bidx * p.nt + t]);
    if (MASK & 2) {
      __syncthreads();  // previous tile's LDS reads are done before flags change
      if (lane == 0) flags[wave] = cls;
      __syncthreads();
      const int any = flags[0] | flags[1] | flags[2] | flags[3];
      if (!any) continue;
    } else if (cls == 0) {
      continue;  // workgroup-uniform (tile mask only)
    }
    const bool oob = (int64_t)(t + 1) * 64 > p.n;
    const bool elem_mask = oob || cls == 2;

    // ---- stage tile t in LDS ------------------------------------------------
    __syncthreads();
    {
      const uint4* ksrc = reinterpret_cast<const uint4*>(kg + (int64_t)t * 64 * D);
      uint4* kdst = reinterpret_cast<uint4*>(smem);
#pragma unroll
      for (int i = tid; i < 4 * D; i += 256) kdst[i] = ksrc[i];
      constexpr int VCH = (PV == kPV_FP8 ? 4 : 8) * D;
      const uint4* vsrc = reinterpret_cast<const uint4*>(vg + (int64_t)t * (VCH * 16));
      uint4* vdst = reinterpret_cast<uint4*>(smem + S::offV);
#pragma unroll
      for (int i = tid; i < VCH; i += 256) vdst[i] = vsrc[i];
      if (GRAN == kGRAN_TOKEN && tid < 16)
        reinterpret_cast<uint4*>(smem + S::offKd)[tid] =
            reinterpret_cast<const uint4*>(p.ks + (int64_t)bh * p.np + (int64_t)t * 64)[tid];
      if (PV == kPV_FP8 && tid >= 64 && tid < 64 + D / 4)
        reinterpret_cast<uint4*>(smem + S::offVd)[tid - 64] =
            reinterpret_cast<const uint4*>(p.vs + ((int64_t)bh * (p.np / 64) + t) * D)[tid - 64];
      if ((MASK & 2) && tid >= 128 && tid < 144) {
        int4 dv;
        const int64_t base = (int64_t)t * 64 + (tid - 128) * 4;
        const int32_t* dsrc = p.doc + (int64_t)bidx * p.n;
        dv.x = base + 0 < p.n ? dsrc[base + 0] : -1;
        dv.y = base + 1 < p.n ? dsrc[base + 1] : -1;
        dv.z = base + 2 < p.n ? dsrc[base + 2] : -1;
        dv.w = base + 3 < p.n ? dsrc[base + 3] : -1;
        reinterpret_cast<int4*>(smem + S::offDoc)[tid - 128] = dv;
      }
    }
    __syncthreads();
    if (cls == 0) continue;

    // ---- S^T = K . Q^T ----------------------------------------------------
    float u[2][16];
    if (QK == kQK_INT8) {
      const i32x4* kl = reinterpret_cast<const i32x4*>(smem);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        i32x16 acc = i32x16{0};
#pragma unroll
        for (int c = 0; c < NC; ++c)
          acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kl[(b * NC + c) * 64 + lane], qf[c], acc, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; ++e) u[b][e] = (float)acc[e];
      }
    } else {
      const i32x4* kl = reinterpret_cast<const i32x4*>(smem);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        f32x16 acc = f32x16{0};
#pragma unroll
        for (int c = 0; c < NC; c += 2) {
          const i32x4 a0 = kl[(b * NC + c) * 64 + lane], a1 = kl[(b * NC + c + 1) * 64 + lane];
          const i32x8 a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
          const i32x8 bq = {qf[c][0], qf[c][1], qf[c][2], qf[c][3],
                            qf[c + 1][0], qf[c + 1][1], qf[c + 1][2], qf[c + 1][3]};
          acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bq, acc, 0, 0, 0, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) u[b][e] = acc[e];
      }
    }

    // ---- per-key scale, masks, row max --------------------------------------
    float w;  // multiplier taking u to log2-domain scores
    if (GRAN == kGRAN_TOKEN) {
      const f32x4* kdl = reinterpret_cast<const f32x4*>(smem + S::offKd);
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 kd4 = kdl[(32 * b + 8 * j + 4 * h) / 4];
#pragma unroll
          for (int i = 0; i < 4; ++i) u[b][4 * j + i] *= kd4[i];
        }
      w = fmaxf(qd, 1e-30f);
    } else {
      w = fmaxf(qd * p.ks[(int64_t)bh * (p.np / 64) + t], 1e-30f);
    }
    if (elem_mask) {
      const int4* dkl = reinterpret_cast<const int4*>(smem + S::offDoc);
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          int4 dk4 = make_int4(0, 0, 0, 0);
          if ((MASK & 2) && cls == 2) dk4 = dkl[(32 * b + 8 * j + 4 * h) / 4];
          const int dk[4] = {dk4.x, dk4.y, dk4.z, dk4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int64_t key = (int64_t)t * 64 + 32 * b + 8 * j + 4 * h + i;
            bool vis = key < p.n;
            if ((MASK & 2) && cls == 2) vis = vis && dk[i] >= 0 && (dq == dk[i] || dq < 0);
            if (!vis) u[b][4 * j + i] = -INFINITY;
          }
        }
    }
    float mu_ = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) mu_ = fmaxf(mu_, u[b][e]);
    mu_ = fmaxf(mu_, __shfl_xor(mu_, 32));
    const float bm = mu_ * w;  // row max of the scores in this tile (-inf if none visible)

    // ---- lazy reference-point update --------------------------------------
    const bool move = (bm > m_ref + kTau) || (m_ref == -INFINITY && bm > -INFINITY);
    float alpha = 1.0f;
    if (move) {
      alpha = exp2f(m_ref - bm);  // 0 when m_ref = -inf
      m_ref = bm;
      l_acc *= alpha;
    }
    if (__any(move)) {
      // O holds rows 8j+4h+i in lane (h, r): fetch those rows' alpha.
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = __shfl(alpha, 8 * j + 4 * h + i);
#pragma unroll
          for (int c = 0; c < NC; ++c) o[c][4 * j + i] *= a;
        }
    }

    // ---- P = 2^(s - m_ref) (scaled), row sums -------------------------------
    const float bias = (m_ref == -INFINITY) ? 0.0f : (c0 - m_ref);
    float pr[2][16];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        pr[b][e] = __builtin_amdgcn_exp2f(fmaf(u[b][e], w, bias));
        l_acc += pr[b][e];
      }

    // ---- O += P . V ---------------------------------------------------------
    if (PV == kPV_FP8) {
      i32x8 pa;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pa[4 * b + j] = (int)pack_fp8x4(pr[b][4 * j], pr[b][4 * j + 1], pr[b][4 * j + 2], pr[b][4 * j + 3]);
      const i32x4* vl = reinterpret_cast<const i32x4*>(smem + S::offV);
      const float* vdl = reinterpret_cast<const float*>(smem + S::offVd);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const i32x4 b0 = vl[(c * 2 + 0) * 64 + lane], b1 = vl[(c * 2 + 1) * 64 + lane];
        const i32x8 bv = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        const f32x16 part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(pa, bv, f32x16{0}, 0, 0, 0, 0, 0, 0);
        const float vd = vdl[32 * c + r];
#pragma unroll
        for (int e = 0; e < 16; ++e) o[c][e] = fmaf(part[e], vd, o[c][e]);
      }
    } else {
      bf16x8 pa[2][2];
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int e = 0; e < 8; ++e) pa[b][tt][e] = (__bf16)pr[b][8 * tt + e];
      const bf16x8* vl = reinterpret_cast<const bf16x8*>(smem + S::offV);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
            o[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[b][tt], vl[((c * 2 + b) * 2 + tt) * 64 + lane], o[c],
                                                           0, 0, 0);
    }
  }

  // ---- epilogue: LSE, normalize, store ---------------------------------------
  const float l_tot = l_acc + __shfl_xor(l_acc, 32);
  const bool empty = !(l_tot > 0.0f);
  const float inv_l = empty ? 0.0f : 1.0f / l_tot;
  if (h == 0 && q0 + r < p.n)
    p.lse[(int64_t)bh * p.n + q0 + r] = empty ? -INFINITY : (m_ref + log2f(l_tot) - c0);
  if (h == 0) xch[r] = inv_l;
  __syncthreads();
  uint16_t* ob = p.out + ((int64_t)bh * p.n + q0) * D;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 8 * j + 4 * h + i;
      const float s = xch[row];
      if (q0 + row < p.n) {
#pragma unroll
        for (int c = 0; c < NC; ++c) ob[(int64_t)row * D + 32 * c + r] = f32_to_bf16_rne(o[c][4 * j + i] * s);
      }
    }
}

// int32 QK^T of int8 codes through the attention kernel's MFMA fragments.
// grid (Np/128, BH, Np/64); wave w covers queries [128*x + 32*w, +32), keys of tile z.
template <int D>
__global__ void __launch_bounds__(256) qk_int32_kernel(const uint8_t* __restrict__ qc, const uint8_t* __restrict__ kc,
                                                       int64_t np, int32_t* __restrict__ s_out) {
  constexpr int NC = D / 32;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, r = lane & 31;
  const int bh = blockIdx.y, t = blockIdx.z;
  const int64_t q0 = (int64_t)blockIdx.x * kRowsPerWG + 32 * wave;
  const uint8_t* qb = qc + (int64_t)bh * np * D + (q0 >> 5) * (32 * D);
  const i32x4* kl = reinterpret_cast<const i32x4*>(kc + (int64_t)bh * np * D + (int64_t)t * 64 * D);
  i32x4 qf[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const i32x4*>(qb + (c * 64 + lane) * 16);
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    i32x16 acc = i32x16{0};
#pragma unroll
    for (int c = 0; c < NC; ++c) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kl[(b * NC + c) * 64 + lane], qf[c], acc, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t key = (int64_t)t * 64 + 32 * b + 8 * j + 4 * h + i;
        s_out[((int64_t)bh * np + q0 + r) * np + key] = acc[4 * j + i];
      }
  }
}

template <int D, int QK, int PV, int GRAN>
hipError_t launch_attn_g(int mask, const AttnParams& p, int64_t bh, hipStream_t st) {
  const dim3 grid((unsigned)(p.np / kRowsPerWG), (unsigned)bh);
  switch (mask) {
    case 0: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 0>), grid, dim3(256), 0, st, p); break;
    case 1: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 1>), grid, dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 2>), grid, dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 3>), grid, dim3(256), 0, st, p); break;
  }
  return hipGetLastError();
}

template <int D>
hipError_t launch_attn_d(int qk, int pv, int gran, int mask, const AttnParams& p, int64_t bh, hipStream_t st) {
#define SAGE_A_CASE(QK_, PV_, G_) \
  if (qk == QK_ && pv == PV_ && gran == G_) return launch_attn_g<D, QK_, PV_, G_>(mask, p, bh, st);
  SAGE_A_CASE(0, 0, 0) SAGE_A_CASE(0, 0, 1) SAGE_A_CASE(0, 1, 0) SAGE_A_CASE(0, 1, 1)
  SAGE_A_CASE(1, 0, 0) SAGE_A_CASE(1, 0, 1) SAGE_A_CASE(1, 1, 0) SAGE_A_CASE(1, 1, 1)
#undef SAGE_A_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_attn(int qk, int pv, int gran, int mask, const AttnParams& p, int64_t bh, int64_t d, int nb,
                       hipStream_t st) {
  if (mask & 2) {
    const int64_t total = (int64_t)nb * (p.nt + p.np / 32);
    hipLaunchKernelGGL(doc_summary_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p.doc, p.n,
                       p.np, nb, p.nt, const_cast<int4*>(p.kv_sum), const_cast<int4*>(p.q_sum));
  }
  if (d == 128) return launch_attn_d<128>(qk, pv, gran, mask, p, bh, st);
  if (d == 64) return launch_attn_d<64>(qk, pv, gran, mask, p, bh, st);
  return hipErrorInvalidValue;
}

hipError_t launch_qk_int32(const uint8_t* qc, const uint8_t* kc, int64_t bh, int64_t n, int64_t d, int32_t* s,
                           hipStream_t st) {
  const int64_t np = padded_len(n);
  const dim3 grid((unsigned)(np / kRowsPerWG), (unsigned)bh, (unsigned)(np / 64));
  if (d == 128)
    hipLaunchKernelGGL(qk_int32_kernel<128>, grid, dim3(256), 0, st, qc, kc, np, s);
  else if (d == 64)
    hipLaunchKernelGGL(qk_int32_kernel<64>, grid, dim3(256), 0, st, qc, kc, np, s);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

size_t attn_workspace_bytes(int64_t b, int64_t n) {
  const int64_t np = padded_len(n);
  const int64_t nt = (n + 63) / 64;
  return (size_t)(b * (nt + np / 32)) * sizeof(int4);
}

}  // namespace sage
