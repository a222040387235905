// Sage attention backward for gfx950 (CDNA4).
//
// Reference: the Triton kernels of sqcu/futudiffu src/futudiffu/sage_kernels.py:
// the D pre-pass _sage_attn_d_prepass (:321-349), dK/dV
// _sage_attn_bwd_dkdv_int8 (:805-916) and its tile-masked form (:1491-1615),
// dQ _sage_attn_bwd_dq_int8 (:918-1030) and its tile-masked form (:1617-1722),
// the fp8-QK kernels (:356-590); launchers sage_attention.py:344-458, :534-648.
//
// Operands.  P is recomputed from the forward's per-token codes exactly as the
// forward scores them, s = acc * qd * kd (qd carrying sm_scale*log2(e)),
// p = 2^(s - lse) with the forward's base-2 LSE.  The quantization kernel
// supplies the Q and smoothed-K codes and scales and, given dO in place of V,
// the T image of dO; one preparation launch (bwd_prep_kernel) writes the T
// images of Q and K~, the R images of dO and V and D = rowsum(dO * O).
//
// T image of bf16 rows X [N, D]: per 64-token block, chunks (j, b, tt) of 64
// lanes x 8 bf16, element 4jj + i of lane 32hh + r holding
// X[32b + 16tt + 8jj + 4hh + i][32j + r].  It is the operand of
// v_mfma_f32_32x32x16_bf16 for a contraction over tokens whose other operand
// comes straight from a 32x32 accumulator (lane (h, r) holding rows
// 8J + 4h + i, element 4J + i): lane half h supplies the same 8 tokens to both
// operands.  The forward's bf16 V operand is the T image of V.
// R image: per 32-token block and 16-channel group, lane (h, r) holds the 16
// bytes X[r][8h, +8) of the group: the row operand of the same instruction for
// a contraction over channels.
//
// Workgroups have 8 waves, two per SIMD; stages pass through a two-stage LDS
// ring filled by direct global -> LDS loads issued one stage ahead (one
// barrier per stage).  Work items are dealt to XCDs in contiguous ranges.
// One launch (bwd_kernel) runs the dK/dV items, then the dQ items.
//
// dQ pass: a workgroup is the forward's 128-query tile; wave w takes queries
// 32 (w % 4) and key half w / 4 of every 64-key tile.  Per wave and tile, in
// the S^T layout (lane (h, r) = query r, keys 8J + 4h + i):
//   S^T = K . Q^T (int8 / fp8 MFMA, the forward's operands),
//   dP^T = V . dO^T (bf16 MFMA; V from the stage, the wave's dO rows in registers),
//   dS^T = P^T (dP^T - D), dQ += dS . K~ (A = dS from the registers, B = T image of K~);
// the two key halves' dQ are added, then dQ * sm_scale is rounded to bf16
// (sage_kernels.py:1720).
// dK/dV pass: a workgroup owns 128 keys; wave w takes keys 32 (w % 4) and
// query half w / 4 of every 64-query step.  Per wave and step, in the S
// layout (lane (h, r) = key r, queries 8J + 4h + i):
//   S = Q . K^T and dP = dO . V^T (the wave's K codes in registers, the
//   workgroup's V rows in LDS for the whole launch),
//   dS = P (dP - D), dV^T += dO^T . bf16(P), dK^T += Q^T . bf16(dS * sm_scale)
// (A = the T images of dO and Q, B = P and dS from the registers); the two
// query halves' dK and dV are added at the end.
// Both kernels skip (query tile, key tile) pairs the reference tile mask turns
// off; with document ids they skip pairs whose summaries show no visible pair
// and give hidden pairs p = 0.
#include <type_traits>

#include "sage_common.h"
#include "sage_launch.h"

namespace sage {

namespace {

__device__ __forceinline__ uint32_t word_at(const uint4& w, int i) {
  return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
}

__device__ __forceinline__ uint4 zero_if(bool z, uint4 w) { return z ? make_uint4(0, 0, 0, 0) : w; }

// 16-byte unit as a native vector: its copies are plain loads and stores.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int QK>
struct BAcc {
  using type = f32x16;
};
template <>
struct BAcc<kQK_INT8> {
  using type = i32x16;
};

// One 32x32 score block from code fragments: rows from `a` (A operand), columns
// from `b`, contracting the D channels (chunks of 32).
template <int D, int QK>
__device__ __forceinline__ typename BAcc<QK>::type score_block(const i32x4* a, const i32x4* b) {
  constexpr int NC = D / 32;
  if constexpr (QK == kQK_INT8) {
    i32x16 acc = i32x16{0};
#pragma unroll
    for (int c = 0; c < NC; ++c) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[c], b[c], acc, 0, 0, 0);
    return acc;
  } else {
    f32x16 acc = f32x16{0};
#pragma unroll
    for (int c = 0; c < NC; c += 2) {
      const i32x8 aa = {a[c][0], a[c][1], a[c][2], a[c][3], a[c + 1][0], a[c + 1][1], a[c + 1][2], a[c + 1][3]};
      const i32x8 bb = {b[c][0], b[c][1], b[c][2], b[c][3], b[c + 1][0], b[c + 1][1], b[c + 1][2], b[c + 1][3]};
      acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aa, bb, acc, 0, 0, 0, 0, 0, 0);
    }
    return acc;
  }
}

__device__ __forceinline__ bool doc_visible(int dq, int dk) { return dk >= 0 && (dq == dk || dq < 0); }

}  // namespace

// ---------------------------------------------------------------------------
// Preparation
// ---------------------------------------------------------------------------

// T image of 64-token block bx of head bh of job z (of up to two bf16
// [BH, N, D] tensors), rows past N zero.  With mu set, the rows are
// bf16(x - mu) (the quantization's smoothed K, sage_attention.py:63-71).
// img: 2 * 64 * D bytes of LDS.
template <int D>
__device__ __forceinline__ void timage_block(const TImageJobs& jobs, int z, int bh, int64_t bx, int64_t n, int64_t np,
                                             uint8_t* img) {
  constexpr int LPR = D / 8;
  constexpr int VTHREADS = 16 * LPR;  // 16 groups of 4 tokens
  const int tid = threadIdx.x;
  const int64_t tok0 = bx * 64;
  const uint16_t* x = jobs.x[z] + (int64_t)bh * n * D;
  const uint16_t* mu = jobs.mu[z];
  if (tid < VTHREADS) {
    const int g = tid / LPR, c8 = tid % LPR;
    uint4 w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t tok = tok0 + 4 * g + i;
      w[i] = zero_if(tok >= n, *reinterpret_cast<const uint4*>(x + min(tok, n - 1) * D + c8 * 8));
    }
    float m8[8];
    if (mu) {
      const uint4 mw = *reinterpret_cast<const uint4*>(mu + (int64_t)bh * D + c8 * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) m8[e] = bf16_to_f32((uint16_t)(word_at(mw, e >> 1) >> ((e & 1) * 16)));
    }
    const int b = g >> 3, tt = (g >> 2) & 1, jj = (g >> 1) & 1, hh = g & 1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = c8 * 8 + e, j = d >> 5, r = d & 31;
      uint32_t t4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t u = (word_at(w[i], e >> 1) >> ((e & 1) * 16)) & 0xffffu;
        if (mu && tok0 + 4 * g + i < n) u = f32_to_bf16_rne(bf16_to_f32((uint16_t)u) - m8[e]);
        t4[i] = u;
      }
      uint2 pk;
      pk.x = t4[0] | (t4[1] << 16);
      pk.y = t4[2] | (t4[3] << 16);
      *reinterpret_cast<uint2*>(img + (((((j * 2 + b) * 2 + tt) * 64 + 32 * hh + r) * 8) + 4 * jj) * 2) = pk;
    }
  }
  __syncthreads();
  uint4* o = reinterpret_cast<uint4*>(jobs.out[z] + ((int64_t)bh * np + tok0) * D);
#pragma unroll
  for (int i = tid; i < 64 * D * 2 / 16; i += 256) o[i] = reinterpret_cast<const uint4*>(img)[i];
}

// R images of up to two bf16 [BH, N, D] tensors (grid.z selects the job): per
// 32-token block rb, 16-channel group c2 and lane L = 32h + r, the 16 bytes
// X[32 rb + r][16 c2 + 8h, +8) at chunk (rb * D/16 + c2) * 64 + L, rows past N
// zero.  It is the row operand of v_mfma_f32_32x32x16_bf16 contracting the
// channels (lane (h, r) = row r, channels 8h.. of the 16-channel step), so a
// stage is a contiguous copy and a fragment read is one 16-byte load per lane.
// One 64-token block (bx) of head bh of job z, one thread per chunk.
template <int D>
__device__ __forceinline__ void rimage_block(const TImageJobs& jobs, int z, int bh, int64_t bx, int64_t n,
                                             int64_t np) {
  constexpr int G = D / 16;           // 16-channel groups
  constexpr int kChunks = 64 * D / 8;  // 16-byte chunks of a 64-token block
  const int64_t tok0 = bx * 64;
  const uint16_t* x = jobs.x[z] + (int64_t)bh * n * D;
  uint4* o = reinterpret_cast<uint4*>(jobs.out[z] + ((int64_t)bh * np + tok0) * D);
#pragma unroll
  for (int c = threadIdx.x; c < kChunks; c += 256) {
    const int lane = c & 63, g = (c >> 6) % G, rb = (c >> 6) / G;
    const int64_t row = tok0 + 32 * rb + (lane & 31);
    const uint4 w = *reinterpret_cast<const uint4*>(x + min(row, n - 1) * D + 16 * g + 8 * (lane >> 5));
    o[c] = zero_if(row >= n, w);
  }
}

// Item of workgroup b of a 1D grid of `total` items: the hardware hands
// workgroup b to XCD b % 8, and each XCD has its own L2, so every XCD takes a
// contiguous range of items (head-major order) and its resident workgroups
// share one head's operands.
__device__ __forceinline__ int xcd_item(int b, int total) {
  constexpr int kXcd = 8;
  const int x = b % kXcd, local = b / kXcd, per = total / kXcd, rem = total % kXcd;
  return x * per + min(x, rem) + local;
}

// D = rowsum(dO * O) per token in fp32 (sage_kernels.py:321-349), zero past N.
// Lane (rr, c8) holds channels [8*c8, +8) of tokens rr + RPP*ps; the products
// are fp32, summed per lane then over the token's lanes.  One 64-token
// block (bx) of head bh.
template <int D>
__device__ __forceinline__ void delta_block(const uint16_t* __restrict__ dout, const uint16_t* __restrict__ out,
                                            int bh, int64_t bx, int64_t n, int64_t np, float* __restrict__ delta) {
  constexpr int LPR = D / 8, RPP = 256 / LPR, PASSES = 64 / RPP;
  const int tid = threadIdx.x, c8 = tid % LPR, rr = tid / LPR;
  const int64_t tok0 = bx * 64;
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int64_t t = tok0 + rr + ps * RPP;
    const int64_t row = ((int64_t)bh * n + min(t, n - 1)) * D + c8 * 8;
    const uint4 a = *reinterpret_cast<const uint4*>(dout + row);
    const uint4 o = *reinterpret_cast<const uint4*>(out + row);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sh = (e & 1) * 16;
      s += bf16_to_f32((uint16_t)(word_at(a, e >> 1) >> sh)) * bf16_to_f32((uint16_t)(word_at(o, e >> 1) >> sh));
    }
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) s += __shfl_xor(s, off);
    if (c8 == 0) delta[(int64_t)bh * np + t] = t < n ? s : 0.0f;
  }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------

// LDS stage of one 64-key tile: K codes (row fragments, as stored), the R
// image of V, the T image of K~, per-key K scales, per-key document ids.
template <int D>
struct DqStage {
  static constexpr int kcBytes = 64 * D;
  static constexpr int rowBytes = 64 * 2 * D;
  static constexpr int offV = kcBytes;
  static constexpr int offT = offV + rowBytes;
  static constexpr int offKd = offT + rowBytes;
  static constexpr int offDoc = offKd + 256;
  static constexpr int bytes = offDoc + 256;
  static constexpr int cKc = kcBytes / 16, cRow = rowBytes / 16;  // 16-byte chunks
};

// Threads of the backward workgroups: 8 waves, two per SIMD, so one wave's
// vector work overlaps the other's matrix and LDS work.
constexpr int kBwdThreads = 512;

// Direct global -> LDS copies by the 8 waves of a backward workgroup.
template <int C, typename Src>
__device__ __forceinline__ void dma_chunks(uint8_t* lds, int wave, int lane, Src src) {
  sage::dma_chunks<C, kBwdThreads / 64>(lds, wave, lane, src);
}

// dQ of item (bh, 128-query tile), in `smem` (2 * DqStage<D>::bytes).  Wave
// w covers queries 32 * (w % 4) of the tile and key half w / 4 of every
// 64-key tile; the two key halves' partial dQ are summed (half 0 + half 1) at
// the end.
// Key tiles [t_begin, t_end) of the item; with cut >= 0 the item is cut item
// `cut` (AttnParams-style in-kernel merge): the half's fp32 dQ goes to its
// slot, and the last half to arrive sums both slots (first half + second
// half) and stores dQ.
template <int D, int QK, int MASK>
__device__ __forceinline__ void dq_item(const BwdParams& p, uint8_t* smem, int item, int t_begin, int t_end,
                                        int cut, int half) {
  using St = DqStage<D>;
  using SAcc = typename BAcc<QK>::type;
  constexpr int NC = D / 32, CPR = D / 8;
  static_assert(4 * NC * 16 * 64 * 4 <= 2 * St::bytes, "partial dQ exchange must fit in the ring");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int h = lane >> 5, r = lane & 31;
  const int qg = wave & 3, b = wave >> 2;  // query group, key half
  const int nq = (int)(p.np / kRowsPerWG);
  const int bh = item / nq, qt = item % nq;
  const int bidx = bh / p.h;
  const int64_t n = p.n, np = p.np;
  const int nt = (int)((n + 63) / 64);
  const int64_t q0 = (int64_t)qt * kRowsPerWG + 32 * qg;
  const bool wave_live = q0 < n;
  const int64_t qrow = q0 + r;

  // ---- per-wave query state -----------------------------------------------------
  i32x4 qf[NC];
  {
    const uint8_t* qb = p.qc + ((int64_t)bh * np + q0) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const i32x4*>(qb + (c * 64 + lane) * 16);
  }
  bf16x8 dof[2 * NC];  // dO[qrow][16c2 + 8h, +8)
  {
    const uint16_t* dr = p.dout + ((int64_t)bh * n + min(qrow, n - 1)) * D + 8 * h;
#pragma unroll
    for (int c2 = 0; c2 < 2 * NC; ++c2) dof[c2] = *reinterpret_cast<const bf16x8*>(dr + 16 * c2);
  }
  const float qd = p.qs[(int64_t)bh * np + qrow];
  // +inf for rows with no gradient (past N, or no visible key in the forward):
  // 2^(s - inf) = 0 needs no per-element test
  const float lse_r = qrow < n ? p.lse[(int64_t)bh * n + qrow] : -INFINITY;
  const float lse_b = lse_r > -INFINITY ? lse_r : INFINITY;
  const float dl = p.delta[(int64_t)bh * np + qrow];
  const int dq_doc = (MASK & 2) ? (qrow < n ? p.doc[(int64_t)bidx * n + qrow] : -1) : 0;
  f32x16 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = f32x16{0};

  // document-id summaries: the workgroup's 128 queries and this wave's 32
  int4 qsum128 = make_int4(0, 0, 0, 0), qsum32 = make_int4(0, 0, 0, 0);
  if constexpr (MASK & 2) {
    qsum128 = p.q_sum128[(int64_t)bidx * nq + qt];
    qsum32 = p.q_sum[(int64_t)bidx * (np / 32) + (q0 >> 5)];
  }
  auto active = [&](int t) __attribute__((always_inline)) -> bool {
    bool on = true;
    if constexpr (MASK & 1)
      on = load_uniform_u8(p.tile_mask, (int64_t)bh * p.mask_stride_z + (int64_t)qt * p.mask_nkv + t) != 0;
    if constexpr (MASK & 2) on = on && classify(qsum128, load_uniform(p.kv_sum, (int64_t)bidx * nt + t)) != 0;
    return on;
  };
  auto next_active = [&](int t) __attribute__((always_inline)) -> int {
    while (t < t_end && !active(t)) ++t;
    return t;
  };

  // ---- staging: bulk by direct global -> LDS loads, scales / ids through registers ----
  u32x4 psm = u32x4{0, 0, 0, 0};
  auto load_tile = [&](int t, int stage) __attribute__((always_inline)) {
    const int64_t key0 = (int64_t)t * 64;
    uint8_t* sb = smem + stage * St::bytes;
    const uint8_t* kcs = p.kc + ((int64_t)bh * np + key0) * D;
    const uint8_t* tks = reinterpret_cast<const uint8_t*>(p.tk + ((int64_t)bh * np + key0) * D);
    const uint8_t* rvs = reinterpret_cast<const uint8_t*>(p.rv + ((int64_t)bh * np + key0) * D);
    if (tid < 32) {
      // one path for lanes 0..31 (see the dK/dV kernel): K scales (g=0),
      // key document ids (g=1, -1 past N)
      const int g = tid >> 4;
      const int64_t k = key0 + 4 * (tid & 15);
      const uint32_t* base = g == 0 ? reinterpret_cast<const uint32_t*>(p.ks + (int64_t)bh * np)
                             : (MASK & 2) ? reinterpret_cast<const uint32_t*>(p.doc + (int64_t)bidx * n)
                                          : reinterpret_cast<const uint32_t*>(p.ks);  // not read
      const int64_t lim = g == 0 ? np : (MASK & 2) ? n : 0;
      const uint32_t dflt = g == 1 ? 0xffffffffu : 0u;
      u32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = k + i < lim ? base[k + i] : dflt;
      psm = v;
    }
    // the stage loads after the small ones (see the dK/dV kernel)
    dma_chunks<St::cKc>(sb, wave, lane, [&](int x) { return kcs + (uint32_t)(x * 16); });
    dma_chunks<St::cRow>(sb + St::offT, wave, lane, [&](int x) { return tks + (uint32_t)(x * 16); });
    dma_chunks<St::cRow>(sb + St::offV, wave, lane, [&](int x) { return rvs + (uint32_t)(x * 16); });
  };
  auto store_small = [&](int stage) __attribute__((always_inline)) {
    uint8_t* sb = smem + stage * St::bytes;
    if (tid < 16)
      reinterpret_cast<u32x4*>(sb + St::offKd)[tid] = psm;
    else if ((MASK & 2) && tid < 32)
      reinterpret_cast<u32x4*>(sb + St::offDoc)[tid - 16] = psm;
  };

  int t = next_active(t_begin);
  if (t < t_end) {
    load_tile(t, 0);
    store_small(0);
  }
  wait_vmem();
  __syncthreads();
  int stage = 0;
  while (t < t_end) {
    const int tn = next_active(t + 1);
    if (tn < t_end) load_tile(tn, stage ^ 1);
    bool wave_on = wave_live;
    if constexpr (MASK & 2)
      wave_on = wave_on && classify(qsum32, load_uniform(p.kv_sum, (int64_t)bidx * nt + t)) != 0;
    if (wave_on) {
      const uint8_t* sb = smem + stage * St::bytes;
      // S^T = K . Q^T for keys 32b + (lane-local rows) x this wave's queries
      i32x4 ka[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) ka[c] = reinterpret_cast<const i32x4*>(sb)[(b * NC + c) * 64 + lane];
      const SAcc s = score_block<D, QK>(ka, qf);
      // dP^T = V . dO^T
      f32x16 dp = f32x16{0};
      const u32x4* vl = reinterpret_cast<const u32x4*>(sb + St::offV);
      u32x4 vf[2 * NC];  // V[key 32b + r][16c2 + 8h, +8), read two MFMAs ahead
      vf[0] = vl[(b * 2 * NC + 0) * 64 + lane];
      vf[1] = vl[(b * 2 * NC + 1) * 64 + lane];
#pragma unroll
      for (int c2 = 0; c2 < 2 * NC; ++c2) {
        __builtin_amdgcn_sched_barrier(0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vf[c2]), dof[c2], dp, 0, 0, 0);
        if (c2 + 2 < 2 * NC) vf[c2 + 2] = vl[(b * 2 * NC + c2 + 2) * 64 + lane];
      }
      // P^T, dS^T (bf16, packed as the A operand of dS . K~)
      const f32x4* kdl = reinterpret_cast<const f32x4*>(sb + St::offKd);
      const int4* dkl = reinterpret_cast<const int4*>(sb + St::offDoc);
      const int kmax = (int)min((int64_t)64, n - (int64_t)t * 64);  // valid keys of this tile
      // the K~ operands of dQ += dS . K~, read before the P / dS vector work
      // so their LDS latency hides under it
      const bf16x8* tkl = reinterpret_cast<const bf16x8*>(sb + St::offT);
      bf16x8 tkf[NC][2];
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) tkf[c][tt] = tkl[((c * 2 + b) * 2 + tt) * 64 + lane];
      bf16x8 dsa[2];
      // s - lse = acc * (qd * kd) - lse; keys past N (the last tile only) are
      // hidden by a test taken on that tile alone
      auto scores = [&](auto ragged) __attribute__((always_inline)) {
#pragma unroll
        for (int J = 0; J < 4; ++J) {
          const f32x4 kd4 = kdl[8 * b + 2 * J + h];
          int4 dk4 = make_int4(0, 0, 0, 0);
          if constexpr (MASK & 2) dk4 = dkl[8 * b + 2 * J + h];
          const int dk[4] = {dk4.x, dk4.y, dk4.z, dk4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int e = 4 * J + i;
            float pr = __builtin_amdgcn_exp2f(fmaf((float)s[e], qd * kd4[i], -lse_b));
            if constexpr (decltype(ragged)::value) pr = 32 * b + 8 * J + 4 * h + i < kmax ? pr : 0.0f;
            if constexpr (MASK & 2) pr = doc_visible(dq_doc, dk[i]) ? pr : 0.0f;
            dsa[e >> 3][e & 7] = (__bf16)(pr * (dp[e] - dl));
          }
        }
      };
      if (kmax < 64)
        scores(std::true_type{});
      else
        scores(std::false_type{});
      // dQ += dS . K~ over this key half
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(dsa[tt], tkf[c][tt], acc[c], 0, 0, 0);
    }
    if (tn < t_end) store_small(stage ^ 1);
    wait_vmem();
    __syncthreads();
    stage ^= 1;
    t = tn;
  }

  // ---- epilogue: dQ = (half 0 + half 1) * sm_scale -> bf16 ---------------------------
  // acc lane (h, r) holds channel 32c + r of rows 8J + 4h + i (element 4J + i)
  float* xch = reinterpret_cast<float*>(smem) + qg * NC * 16 * 64;
  if (b == 1) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) xch[(c * 16 + e) * 64 + lane] = acc[c][e];
  }
  __syncthreads();
  if (b == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[c][e] += xch[(c * 16 + e) * 64 + lane];
  }
  __syncthreads();
  if (cut >= 0) {
    // a half of a cut item: its dQ through to the coherence point, complete
    // before it counts; the last half sums the two slots in key order
    constexpr int kSlot = 4 * NC * 16 * 64;
    uint32_t* slots = reinterpret_cast<uint32_t*>(p.dq_part + (int64_t)cut * 2 * kSlot);
    if (b == 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          __hip_atomic_store(slots + half * kSlot + ((qg * NC + c) * 16 + e) * 64 + lane, __float_as_uint(acc[c][e]),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vmem();
    __syncthreads();
    int* last = reinterpret_cast<int*>(smem);
    if (tid == 0) *last = arrive_last(p.dq_ctr + cut, p.dq_tag, 2) ? 1 : 0;
    __syncthreads();
    if (*last == 0) return;
    if (b == 0) {
      auto ld = [](const uint32_t* a) __attribute__((always_inline)) {
        return __uint_as_float(__hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      };
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int at = ((qg * NC + c) * 16 + e) * 64 + lane;
          acc[c][e] = ld(slots + at) + ld(slots + kSlot + at);
        }
    }
    if (tid == 0)
      __hip_atomic_store(p.dq_ctr + cut, p.dq_tag << 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();  // every wave has read `last` before the staging below reuses the LDS
  }
  uint16_t* stg = reinterpret_cast<uint16_t*>(smem) + qg * 32 * D;
  if (b == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = 8 * (e >> 2) + 4 * h + (e & 3);
        stg[row * D + 32 * c + r] = f32_to_bf16_rne(acc[c][e] * p.sm_scale);
      }
  }
  __syncthreads();
  // all 8 waves store: wave w writes half (w / 4) of the rows of query group w % 4
#pragma unroll
  for (int i = 0; i < 16 * CPR / 64; ++i) {
    const int x = 16 * CPR * b + lane + 64 * i, row = x / CPR, ch = x % CPR;
    const int64_t q = q0 + row;
    if (q < n)
      *reinterpret_cast<uint4*>(p.dq + ((int64_t)bh * n + q) * D + ch * 8) =
          reinterpret_cast<const uint4*>(stg)[x];
  }
}

// ---------------------------------------------------------------------------
// dK, dV
// ---------------------------------------------------------------------------

// LDS stage of one 64-query step: Q codes (row fragments), the R image of dO,
// T images of dO and Q, per-query Q scale, LSE (+inf for rows without
// gradient), D, document ids.
template <int D>
struct DkvStage {
  static constexpr int qcBytes = 64 * D;
  static constexpr int rowBytes = 64 * 2 * D;
  static constexpr int offDo = qcBytes;
  static constexpr int offTdo = offDo + rowBytes;
  static constexpr int offTq = offTdo + rowBytes;
  static constexpr int offQd = offTq + rowBytes;
  static constexpr int offLse = offQd + 256;
  static constexpr int offDl = offLse + 256;
  static constexpr int offDoc = offDl + 256;
  static constexpr int bytes = offDoc + 256;
  static constexpr int cQc = qcBytes / 16, cRow = rowBytes / 16;
};

// LDS of a dK/dV item: two step stages, then the R image of the workgroup's
// 128 V rows, read as the B operand of dP by the waves that own them.
template <int D>
constexpr int kDkvLds = 2 * DkvStage<D>::bytes + kRowsPerWG * 2 * D;

// dK, dV of item (bh, 128-key block), in `smem` (kDkvLds<D>).  Wave w owns
// keys 32 * (w % 4) of the workgroup's 128 keys and query half w / 4 of every
// 64-query step; the two query halves' partial dK and dV are summed (half 0 +
// half 1) at the end.
template <int D, int QK, int MASK>
__device__ __forceinline__ void dkdv_item(const BwdParams& p, uint8_t* smem, int item) {
  using St = DkvStage<D>;
  using SAcc = typename BAcc<QK>::type;
  constexpr int NC = D / 32, CPR = D / 8;
  constexpr int kVOff = 2 * St::bytes;
  static_assert(4 * NC * 16 * 64 * 4 <= 2 * St::bytes, "partial dK/dV exchange must fit in the ring");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int h = lane >> 5, r = lane & 31;
  const int kg = wave & 3, a = wave >> 2;  // key group, query half
  const int nkb = (int)(p.np / kRowsPerWG);
  const int bh = item / nkb, kb = item % nkb;
  const int bidx = bh / p.h;
  const int64_t n = p.n, np = p.np;
  const int nkv = (int)((n + 63) / 64);
  const int nsteps = (int)((n + 63) / 64);  // 64-query steps holding a query below N
  const int64_t k0 = (int64_t)kb * kRowsPerWG + 32 * kg;
  const int64_t krow = k0 + r;
  const int my_tile = 2 * kb + (kg >> 1);  // reference KV tile of this wave's keys
  const bool wave_live = k0 < n;

  // ---- per-wave key state -------------------------------------------------------------
  i32x4 kf[NC];
  {
    const uint8_t* kbp = p.kc + ((int64_t)bh * np + k0) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) kf[c] = *reinterpret_cast<const i32x4*>(kbp + (c * 64 + lane) * 16);
  }
  {
    // the R image of V rows [kb*128, +128) into the persistent region
    const uint8_t* rvs = reinterpret_cast<const uint8_t*>(p.rv + ((int64_t)bh * np + (int64_t)kb * kRowsPerWG) * D);
    dma_chunks<kRowsPerWG * CPR>(smem + kVOff, wave, lane, [&](int x) { return rvs + (uint32_t)(x * 16); });
  }
  const u32x4* vrl = reinterpret_cast<const u32x4*>(smem + kVOff);
  const float kd = p.ks[(int64_t)bh * np + krow];
  const bool key_ok = krow < n;
  const int dk_doc = (MASK & 2) ? (key_ok ? p.doc[(int64_t)bidx * n + krow] : -1) : 0;
  f32x16 dva[NC], dka[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    dva[c] = f32x16{0};
    dka[c] = f32x16{0};
  }

  const uint8_t* mrow = (MASK & 1) ? p.tile_mask + (int64_t)bh * p.mask_stride_z : nullptr;
  // document-id summaries of the workgroup's two key tiles
  const int4* qs32 = (MASK & 2) ? p.q_sum + (int64_t)bidx * (np / 32) : nullptr;
  int4 ksum[2] = {make_int4(0, 0, 0, 0), make_int4(0, 0, 0, 0)};
  if constexpr (MASK & 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      ksum[i] = 2 * kb + i < nkv ? load_uniform(p.kv_sum, (int64_t)bidx * nkv + 2 * kb + i)
                                 : make_int4(0x7fffffff, -0x7fffffff, 0, 0);
  }
  auto wave_active = [&](int s) __attribute__((always_inline)) -> bool {
    bool on = true;
    if constexpr (MASK & 1) on = my_tile < nkv && load_uniform_u8(mrow, (int64_t)(s >> 1) * p.mask_nkv + my_tile) != 0;
    if constexpr (MASK & 2) on = on && classify(load_uniform(qs32, 2 * s + a), ksum[kg >> 1]) != 0;
    return on;
  };
  auto active = [&](int s) __attribute__((always_inline)) -> bool {
    bool on = true;
    if constexpr (MASK & 1) {
      const uint8_t* m = mrow + (int64_t)(s >> 1) * p.mask_nkv;
      on = load_uniform_u8(m, 2 * kb) != 0 || (2 * kb + 1 < nkv && load_uniform_u8(m, 2 * kb + 1) != 0);
    }
    if constexpr (MASK & 2) {
      const int4 q64 = merge_summary(load_uniform(qs32, 2 * s), load_uniform(qs32, 2 * s + 1));
      on = on && (classify(q64, ksum[0]) != 0 || classify(q64, ksum[1]) != 0);
    }
    return on;
  };
  auto next_active = [&](int s) __attribute__((always_inline)) -> int {
    while (s < nsteps && !active(s)) ++s;
    return s;
  };

  // ---- staging: bulk by direct global -> LDS loads, per-query values through registers ----
  u32x4 psm = u32x4{0, 0, 0, 0};
  auto load_step = [&](int s, int stage) __attribute__((always_inline)) {
    const int64_t m0 = (int64_t)s * 64;
    uint8_t* sb = smem + stage * St::bytes;
    const uint8_t* qcs = p.qc + ((int64_t)bh * np + m0) * D;
    const uint8_t* tds = reinterpret_cast<const uint8_t*>(p.tdo + ((int64_t)bh * np + m0) * D);
    const uint8_t* tqs = reinterpret_cast<const uint8_t*>(p.tq + ((int64_t)bh * np + m0) * D);
    const uint8_t* rds = reinterpret_cast<const uint8_t*>(p.rdo + ((int64_t)bh * np + m0) * D);
    if (tid < 64) {
      // one path for the 64 lanes of wave 0 (no per-lane branches writing the
      // same registers, which would make the compiler wait for loads in
      // flight, the stage loads included): lanes 16g .. 16g+15 take values
      // 4(lane&15) .. +3 of the Q scales (g=0), LSE (g=1, -inf past N), D
      // (g=2) or query document ids (g=3, -1 past N)
      const int g = tid >> 4;
      const int64_t m = m0 + 4 * (tid & 15);
      const uint32_t* base = g == 0   ? reinterpret_cast<const uint32_t*>(p.qs + (int64_t)bh * np)
                             : g == 1 ? reinterpret_cast<const uint32_t*>(p.lse + (int64_t)bh * n)
                             : g == 2 ? reinterpret_cast<const uint32_t*>(p.delta + (int64_t)bh * np)
                             : (MASK & 2) ? reinterpret_cast<const uint32_t*>(p.doc + (int64_t)bidx * n)
                                          : reinterpret_cast<const uint32_t*>(p.qs);  // not read
      const int64_t lim = (g == 0 || g == 2) ? np : (g == 1 || (MASK & 2)) ? n : 0;
      const uint32_t dflt = g == 1 ? __float_as_uint(-INFINITY) : g == 3 ? 0xffffffffu : 0u;
      u32x4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = m + i < lim ? base[m + i] : dflt;
      psm = v;
    }
    // the stage loads after the small ones: a wait for the small values then
    // leaves the stage loads in flight
    dma_chunks<St::cQc>(sb, wave, lane, [&](int x) { return qcs + (uint32_t)(x * 16); });
    dma_chunks<St::cRow>(sb + St::offTdo, wave, lane, [&](int x) { return tds + (uint32_t)(x * 16); });
    dma_chunks<St::cRow>(sb + St::offTq, wave, lane, [&](int x) { return tqs + (uint32_t)(x * 16); });
    dma_chunks<St::cRow>(sb + St::offDo, wave, lane, [&](int x) { return rds + (uint32_t)(x * 16); });
  };
  auto store_small = [&](int stage) __attribute__((always_inline)) {
    uint8_t* sb = smem + stage * St::bytes;
    u32x4 v = psm;
    if (tid >= 16 && tid < 32) {
      // +inf for rows with no gradient (past N, or no visible key in the
      // forward): 2^(s - inf) = 0 needs no per-element test
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(v[i]) > -INFINITY ? v[i] : __float_as_uint(INFINITY);
    }
    if (tid < 48 || ((MASK & 2) && tid < 64)) reinterpret_cast<u32x4*>(sb + St::offQd)[tid] = v;
  };

  int s = next_active(0);
  if (s < nsteps) {
    load_step(s, 0);
    store_small(0);
  }
  wait_vmem();
  __syncthreads();
  int stage = 0;
  while (s < nsteps) {
    const int sn = next_active(s + 1);
    if (sn < nsteps) load_step(sn, stage ^ 1);
    if (wave_live && wave_active(s)) {
      const uint8_t* sb = smem + stage * St::bytes;
      const f32x4* qdl = reinterpret_cast<const f32x4*>(sb + St::offQd);
      const f32x4* lsl = reinterpret_cast<const f32x4*>(sb + St::offLse);
      const f32x4* dll = reinterpret_cast<const f32x4*>(sb + St::offDl);
      const int4* dql = reinterpret_cast<const int4*>(sb + St::offDoc);
      const u32x4* dol = reinterpret_cast<const u32x4*>(sb + St::offDo);
      const bf16x8* tdl = reinterpret_cast<const bf16x8*>(sb + St::offTdo);
      const bf16x8* tql = reinterpret_cast<const bf16x8*>(sb + St::offTq);
      // S = Q . K^T: rows = queries 32a + (lane-local rows), columns = this wave's keys
      i32x4 qa[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) qa[c] = reinterpret_cast<const i32x4*>(sb)[(a * NC + c) * 64 + lane];
      const SAcc sacc = score_block<D, QK>(qa, kf);
      // dP = dO . V^T, operands read two MFMAs ahead of their use
      f32x16 dp = f32x16{0};
      u32x4 wf[2 * NC], vf[2 * NC];
      auto dpfrag = [&](int c2) __attribute__((always_inline)) {
        wf[c2] = dol[(a * 2 * NC + c2) * 64 + lane];   // dO[query 32a + r][16c2 + 8h, +8)
        vf[c2] = vrl[(kg * 2 * NC + c2) * 64 + lane];  // V[krow][16c2 + 8h, +8)
      };
      dpfrag(0);
      dpfrag(1);
#pragma unroll
      for (int c2 = 0; c2 < 2 * NC; ++c2) {
        __builtin_amdgcn_sched_barrier(0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wf[c2]),
                                                     __builtin_bit_cast(bf16x8, vf[c2]), dp, 0, 0, 0);
        if (c2 + 2 < 2 * NC) dpfrag(c2 + 2);
      }
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        const f32x4 qd4 = qdl[8 * a + 2 * J + h];
        const f32x4 ls4 = lsl[8 * a + 2 * J + h];
        const f32x4 dl4 = dll[8 * a + 2 * J + h];
        int4 dq4 = make_int4(0, 0, 0, 0);
        if constexpr (MASK & 2) dq4 = dql[8 * a + 2 * J + h];
        const int dqd[4] = {dq4.x, dq4.y, dq4.z, dq4.w};
        // s - lse = acc * (qd * kd) - lse; keys past N need no test: their
        // column only feeds their own dK / dV rows, which are not stored
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * J + i;
          float pr = __builtin_amdgcn_exp2f(fmaf((float)sacc[e], qd4[i] * kd, -ls4[i]));
          if constexpr (MASK & 2) pr = doc_visible(dqd[i], dk_doc) ? pr : 0.0f;
          const float ds = pr * (dp[e] - dl4[i]);
          pb[e >> 3][e & 7] = (__bf16)pr;
          db[e >> 3][e & 7] = (__bf16)(ds * p.sm_scale);
        }
      }
      // dV^T += dO^T . P, dK^T += Q^T . dS over this query half; operand
      // fragments read two MFMA pairs ahead of their use
      constexpr int kPairs = NC * 2, kAhead = 2;
      bf16x8 tdf[kPairs], tqf[kPairs];
      auto frag = [&](int i) __attribute__((always_inline)) {
        const int ci = (((i >> 1) * 2 + a) * 2 + (i & 1)) * 64 + lane;  // c = i / 2, tt = i % 2
        tdf[i] = tdl[ci];
        tqf[i] = tql[ci];
      };
#pragma unroll
      for (int i = 0; i < kAhead; ++i) frag(i);
#pragma unroll
      for (int i = 0; i < kPairs; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        const int c = i >> 1, tt = i & 1;
        dva[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tdf[i], pb[tt], dva[c], 0, 0, 0);
        dka[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tqf[i], db[tt], dka[c], 0, 0, 0);
        if (i + kAhead < kPairs) frag(i + kAhead);
      }
    }
    if (sn < nsteps) store_small(stage ^ 1);
    wait_vmem();
    __syncthreads();
    stage ^= 1;
    s = sn;
  }

  // ---- epilogue: (half 0 + half 1), lane (h, r) holds key r, channels 32c + 8J + 4h + i ----
  float* xch = reinterpret_cast<float*>(smem) + kg * NC * 16 * 64;
  if (a == 1) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) xch[(c * 16 + e) * 64 + lane] = dva[c][e];
  }
  __syncthreads();
  if (a == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) dva[c][e] += xch[(c * 16 + e) * 64 + lane];
  }
  __syncthreads();
  if (a == 1) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) xch[(c * 16 + e) * 64 + lane] = dka[c][e];
  }
  __syncthreads();
  if (a == 0 && key_ok) {
    uint16_t* dvr = p.dv + ((int64_t)bh * n + krow) * D;
    uint16_t* dkr = p.dk + ((int64_t)bh * n + krow) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        const int ch = 32 * c + 8 * J + 4 * h;
        float kk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) kk[i] = dka[c][4 * J + i] + xch[(c * 16 + 4 * J + i) * 64 + lane];
        uint2 va, ka2;
        va.x = f32_to_bf16_rne(dva[c][4 * J + 0]) | ((uint32_t)f32_to_bf16_rne(dva[c][4 * J + 1]) << 16);
        va.y = f32_to_bf16_rne(dva[c][4 * J + 2]) | ((uint32_t)f32_to_bf16_rne(dva[c][4 * J + 3]) << 16);
        ka2.x = f32_to_bf16_rne(kk[0]) | ((uint32_t)f32_to_bf16_rne(kk[1]) << 16);
        ka2.y = f32_to_bf16_rne(kk[2]) | ((uint32_t)f32_to_bf16_rne(kk[3]) << 16);
        *reinterpret_cast<uint2*>(dvr + ch) = va;
        *reinterpret_cast<uint2*>(dkr + ch) = ka2;
      }
  }
}

// The two gradient passes in one launch: workgroups [0, kv_wgs) take the
// dK/dV items (kv_wgs = items rounded up to a multiple of 8, the extra ones
// exit), the next `items` the dQ items, of which the last p.dq_split take the
// first key-tile half of their item, and the dq_split after those the second
// halves (dispatched last, the short pieces fill the launch's end).  The passes are independent, so the
// dQ items fill the CUs the last dK/dV round leaves idle, and the shorter
// items come last.  Each part deals its items to the XCDs like a launch of
// its own (xcd_item): kv_wgs is a multiple of the XCD count, so a dQ
// workgroup's XCD is its index within the part modulo 8.
template <int D>
constexpr int kBwdLds = kDkvLds<D> > 2 * DqStage<D>::bytes ? kDkvLds<D> : 2 * DqStage<D>::bytes;

template <int D, int QK, int MASK>
__global__ void __launch_bounds__(kBwdThreads) bwd_kernel(BwdParams p, int items, int kv_wgs) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kBwdLds<D>];
  const int wg = (int)blockIdx.x;
  const int nt = (int)((p.n + 63) / 64), mid = nt / 2;
  if (wg < kv_wgs) {
    if (wg < items) dkdv_item<D, QK, MASK>(p, smem, xcd_item(wg, items));
    return;
  }
  const int j = wg - kv_wgs, whole = items - p.dq_split;
  if (j < whole)
    dq_item<D, QK, MASK>(p, smem, xcd_item(j, items), 0, nt, -1, 0);
  else if (j < items)
    dq_item<D, QK, MASK>(p, smem, xcd_item(j, items), 0, mid, j - whole, 0);
  else
    dq_item<D, QK, MASK>(p, smem, xcd_item(j - p.dq_split, items), mid, nt, j - items, 1);
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

// The preparation in one launch, grid (np / 64, BH, 5): z = 0, 1 the T images
// of tjobs, z = 2, 3 the R images of rjobs, z = 4 D.
template <int D>
__global__ void __launch_bounds__(256) bwd_prep_kernel(TImageJobs tjobs, TImageJobs rjobs,
                                                       const uint16_t* __restrict__ dout,
                                                       const uint16_t* __restrict__ out, int64_t n, int64_t np,
                                                       float* __restrict__ delta) {
  __shared__ __attribute__((aligned(16))) uint8_t img[2 * 64 * D];
  const int z = blockIdx.z, bh = blockIdx.y;
  const int64_t bx = blockIdx.x;
  if (z < 2)
    timage_block<D>(tjobs, z, bh, bx, n, np, img);
  else if (z < 4)
    rimage_block<D>(rjobs, z - 2, bh, bx, n, np);
  else
    delta_block<D>(dout, out, bh, bx, n, np, delta);
}

hipError_t launch_bwd_prep(const TImageJobs& tjobs, const TImageJobs& rjobs, const uint16_t* dout,
                           const uint16_t* out, int64_t bh, int64_t n, int64_t d, float* delta, hipStream_t st) {
  const int64_t np = padded_len(n);
  const dim3 grid((unsigned)(np / 64), (unsigned)bh, 5u);
  if (d == 128)
    hipLaunchKernelGGL(bwd_prep_kernel<128>, grid, dim3(256), 0, st, tjobs, rjobs, dout, out, n, np, delta);
  else if (d == 64)
    hipLaunchKernelGGL(bwd_prep_kernel<64>, grid, dim3(256), 0, st, tjobs, rjobs, dout, out, n, np, delta);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int D, int QK, int MASK>
hipError_t launch_bwd_t(const BwdParams& p, int64_t bh, hipStream_t st) {
  const int64_t items = p.np / kRowsPerWG * bh;  // per pass, in xcd_item order
  const int64_t kv_wgs = (items + 7) / 8 * 8;
  hipLaunchKernelGGL((bwd_kernel<D, QK, MASK>), dim3((unsigned)(kv_wgs + items + p.dq_split)), dim3(kBwdThreads), 0,
                     st, p, (int)items, (int)kv_wgs);
  return hipGetLastError();
}

template <int D>
hipError_t launch_bwd_d(int qk, int mask, const BwdParams& p, int64_t bh, hipStream_t st) {
#define SAGE_B_CASE(QK_, M_) \
  if (qk == QK_ && mask == M_) return launch_bwd_t<D, QK_, M_>(p, bh, st);
  SAGE_B_CASE(0, 0) SAGE_B_CASE(0, 1) SAGE_B_CASE(0, 2) SAGE_B_CASE(0, 3)
  SAGE_B_CASE(1, 0) SAGE_B_CASE(1, 1) SAGE_B_CASE(1, 2) SAGE_B_CASE(1, 3)
#undef SAGE_B_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_bwd(int qk, int mask, const BwdParams& p, int64_t d, int64_t bh, hipStream_t st) {
  if (d == 128) return launch_bwd_d<128>(qk, mask, p, bh, st);
  if (d == 64) return launch_bwd_d<64>(qk, mask, p, bh, st);
  return hipErrorInvalidValue;
}

}  // namespace sage
