// Fused Sage attention forward for gfx950 (CDNA4).
//
// Reference: the Triton kernels of sqcu/futudiffu src/futudiffu/sage_kernels.py:
// production variant _sage_attn_fwd_int8qk_bf16pv_masked_lse (:1378-1477),
// fp8-QK variants (:215-315) and the fp8 P/V stage of
// _sage_attn_fwd_fp8qk_fp8pv_lse (:1135-1154).
//
// Work decomposition: one workgroup = 4 waves = 128 query rows (the reference
// Q tile, so a reference tile mask is workgroup-uniform); each wave owns 32
// query rows.  Keys stream in 64-key tiles (the reference KV tile, which is
// also the V-scale block) through a ring of LDS stages filled by direct
// global -> LDS loads: tile i+2 is issued while tile i is consumed and tile
// i+1 already feeds the next S^T; one barrier per tile.  Without document
// ids (and with them for fp8 P.V) the loop is software-pipelined: the P.V of
// tile i-1 is formed in iteration i, its MFMAs under tile i's score
// conversion and softmax.
//
// Per wave and tile:
//   S^T[key][query] = K . Q^T with v_mfma_i32_32x32x32_i8 (int8) or
//   v_mfma_f32_32x32x64_f8f6f4 (fp8): lane (h, r) holds query r and keys
//   32b + 8j + 4h + i, so every per-query reduction is lane-local (plus one
//   permlane32 swap between the two lane halves).  The S^T of tile i+1 is
//   issued before the softmax of tile i so the matrix cores and the vector
//   ALUs overlap within the wave.
//   Online softmax in fp32 with exp2 (scores are in log2 units).
//   O[query][d] += P . V with v_mfma_f32_32x32x64_f8f6f4 (fp8 P, fp8 V) or
//   v_mfma_f32_32x32x16_bf16 (bf16 P, bf16 V).  P feeds the MFMA straight
//   from the S^T registers: lane (h, r) already holds the keys its A operand
//   needs.  O lane (h, r) holds channel 32c + r of rows 8j + 4h + i.
//
// O and l are kept in a lazily moved frame: they hold sums of 2^(s - m_ref),
// where the per-row reference point m_ref only moves when a block max exceeds
// it by more than kTau (then O and l are rescaled, which is rare after the
// first tiles).  The LSE is m_ref + log2(l), the reference's m + log2(l).
// fp8 P follows the reference per (row, 64-key block) scaling
// (sage_kernels.py:1137-1141): with bm the block's row max, the code argument
// is e = 2^(s - bm) * 448 (= p * 448 / max(p)), and the block's PV product is
// dequantized by 2^(bm - m_ref) / 448 per row and the V scale per channel
// (the rank-1 factor matrix comes from a small fp32 MFMA).
// bf16 P is 2^(s - m_ref) rounded to bf16; bf16 rounding is relative, so this
// matches the reference's bf16(2^(s - m)) up to exp2 rounding.
#include <algorithm>
#include <type_traits>

#include "sage_common.h"
#include "sage_launch.h"

namespace sage {

// Per-phase timing of the pipelined loop, built only into the measurement
// library (SAGE_PHASE_TIMING; futudiffu_amd/build.py --phase-timing): every
// live wave accumulates s_memtime ticks per phase of each loop iteration
// (scheduling fences keep each phase's instructions inside it) and stores
// them, with its iteration count, to one slot per (workgroup, wave).
#ifdef SAGE_PHASE_TIMING
constexpr int kPhaseSlots = 32768;
constexpr int kPhases = 6;  // slot words 0..5 phases, 6 iterations, 7 ticks in the loop
__device__ unsigned long long sage_phase_buf[kPhaseSlots][8];
#define SAGE_PHASE(k)                                      \
  do {                                                     \
    __builtin_amdgcn_sched_barrier(0);                     \
    const uint64_t now_ = __builtin_amdgcn_s_memtime();    \
    ph_acc[k] += now_ - ph_last;                           \
    ph_last = now_;                                        \
    __builtin_amdgcn_sched_barrier(0);                     \
  } while (0)
#else
#define SAGE_PHASE(k) \
  do {                \
  } while (0)
#endif

constexpr float kLog2Fp8Max = 8.807354922057604f;  // log2(448)
typedef float f32x32 __attribute__((ext_vector_type(32)));

// Per-batch token summaries: kv tiles of 64, query blocks of 32 and of 128.
// One wave per summary (grid-stride over summaries): lane l reads tokens
// t0 + l and t0 + 64 + l, then wave-wide min / max / sums.
__global__ void __launch_bounds__(256) doc_summary_kernel(const int32_t* __restrict__ doc, int64_t n, int64_t np,
                                                          int nb, int nt, int4* __restrict__ kv_sum,
                                                          int4* __restrict__ q_sum, int4* __restrict__ q_sum128,
                                                          int4* __restrict__ heavy) {
  const int64_t nq32 = np / 32, nq128 = np / 128;
  // the list of split query tiles that doc_prefix_kernel fills starts empty
  if (heavy != nullptr && blockIdx.x == 0 && threadIdx.x == 0) heavy[0] = make_int4(0, 0, 0, 0);
  const int lane = threadIdx.x & 63;
  const int64_t per_b = nt + nq32 + nq128;
  const int64_t total = (int64_t)nb * per_b;
  const int64_t stride = (int64_t)gridDim.x * (blockDim.x >> 6);
  // idx is wave-uniform: every lane of a wave runs the same iterations
  for (int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; idx < total; idx += stride) {
    const int b = (int)(idx / per_b);
    const int64_t w = idx % per_b;
    int64_t t0, len;
    int4* dst;
    if (w < nt) {
      t0 = w * 64;
      len = 64;
      dst = kv_sum + (int64_t)b * nt + w;
    } else if (w < nt + nq32) {
      t0 = (w - nt) * 32;
      len = 32;
      dst = q_sum + (int64_t)b * nq32 + (w - nt);
    } else {
      t0 = (w - nt - nq32) * 128;
      len = 128;
      dst = q_sum128 + (int64_t)b * nq128 + (w - nt - nq32);
    }
    int mn = 0x7fffffff, mx = -0x7fffffff, nv = 0, ni = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int64_t i = t0 + 64 * s + lane;
      if (64 * s + lane < len && i < n) {
        const int dd = doc[(int64_t)b * n + i];
        if (dd >= 0) {
          mn = min(mn, dd);
          mx = max(mx, dd);
          ++nv;
        } else {
          ++ni;
        }
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      mn = min(mn, __shfl_xor(mn, off));
      mx = max(mx, __shfl_xor(mx, off));
      nv += __shfl_xor(nv, off);
      ni += __shfl_xor(ni, off);
    }
    if (lane == 0) *dst = make_int4(mn, mx, nv, ni);
  }
}

// LDS stage layout (bytes): K codes, V operand, then a contiguous region of
// per-key K scales (token granularity) and per-channel V scales (fp8 P.V),
// then per-key document ids.  Every part except the document ids arrives by
// direct global -> LDS loads.
template <int D, int PV>
struct Stage {
  static constexpr int kBytes = 64 * D;
  static constexpr int vBytes = (PV == kPV_FP8 ? 64 : 128) * D;
  static constexpr int offV = kBytes;
  static constexpr int offKd = offV + vBytes;
  static constexpr int offVd = offKd + 256;
  static constexpr int offDoc = offVd + (PV == kPV_FP8 ? 4 * D : 0);
  static constexpr int bytes = offDoc + 256;
  static constexpr int cK = kBytes / 16, cV = vBytes / 16;  // 16-byte chunks of the K and V parts
};

// Workgroup LDS: a ring of stages, then a 32-float row exchange per wave.  With
// fp8 P.V four stages: the product of tile i-1 is formed while tile i is
// consumed, tile i+1 feeds the next QK^T and tile i+2 is being written.  With
// bf16 P.V (a stage of 24.5 KB at D = 128) three stages: in the pipelined
// loop a tile's K part is loaded two tiles ahead and the rest one tile ahead,
// so K of tile i+2 shares a stage with V of tile i-1; in the general loop
// tile i is consumed while tile i+1 feeds the next QK^T and tile i+2 is being
// written.  The bf16 output staging of the epilogue reuses the ring.
template <int D, int PV>
struct Smem {
  static constexpr int kStages = PV == kPV_FP8 ? 4 : 3;
  static constexpr int offX = kStages * Stage<D, PV>::bytes;
  static constexpr int bytes = offX + 4 * 32 * 4;
  static_assert(4 * 32 * D * 2 <= offX, "epilogue staging must fit in the stage ring");
};

// Work item of a workgroup: (bh, 128-row query tile).
// The hardware hands workgroup i to XCD i % 8, and each XCD has its own L2.
// Items are therefore dealt to XCDs in contiguous head-major ranges, so the
// workgroups resident on one XCD at a time cover about two heads and their
// K/V tiles stay in that XCD's L2.  When the last query tile of each head
// holds at most 64 rows (two idle waves), those light items come last in every
// XCD's range so the final, partial dispatch round is short.
__device__ __forceinline__ void item_of(int id, int total, int bh_count, int nq, bool light_last, int& bh, int& qt) {
  constexpr int kXcd = 8;
  const int light = (light_last && nq > 1) ? bh_count : 0;  // one light item per head
  const int x = id % kXcd, local = id / kXcd;
  const int per = total / kXcd, rem = total % kXcd;
  const int lper = light / kXcd, lrem = light % kXcd;
  const int count = per + (x < rem ? 1 : 0);
  const int lcount = lper + (x < lrem ? 1 : 0);
  const int lstart = x * lper + min(x, lrem);
  const int hcount = count - lcount;
  const int hstart = x * per + min(x, rem) - lstart;
  const int nqh = light ? nq - 1 : nq;  // heavy tiles per head
  if (local < hcount) {
    const int hi = hstart + local;
    bh = hi / nqh;
    qt = hi % nqh;
  } else {
    bh = lstart + (local - hcount);
    qt = nq - 1;
  }
}

// The start of the int8 QK^T chains.  C0 false: 0, which the MFMA takes as
// an inline C operand (no registers), and a score is float(acc) * kd, exact
// in the conversion since |acc| <= 128 * 127^2 < 2^21.  C0 true: the bit
// pattern of c0 = 1/(2 pi); acc + c0_bits stays inside c0's binade [1/8, 1/4),
// whose ulp is 2^-26, so the accumulator read as fp32 is exactly
// x = c0 + acc * 2^-26 and x - c0 = acc * 2^-26 exactly (Sterbenz): one
// subtraction (issued at about twice the rate of v_cvt_f32_i32) reads the
// sum, and the 2^26 goes into the row multiplier, so scores, maxima and exp
// arguments are the same floats either way.  The compiler keeps that splat
// in 16 registers: the document-id loops gain from the subtraction
// (1x30x6912 packed 363.7 -> 360.4 us, the 4x30x4352 key-padded batch
// 980.9 -> 975.5 us), the others from the registers (1x30x4416x128
// 242.3 -> 241.2 us, the packed tile-mask batch 343.9 -> 334.5 us).
constexpr int32_t kC0Bits = 0x3E22F983;
constexpr float kC0 = 0.15915494309189535f;
static_assert(__builtin_bit_cast(int32_t, kC0) == kC0Bits, "c0 must be the inline constant 1/(2 pi)");
constexpr float kC0Scale = 67108864.0f;  // 2^26, the accumulator's ulp inverted
template <bool C0>
__device__ __forceinline__ i32x16 i8_start() {
  if constexpr (C0)
    return i32x16{kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits,
                  kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits, kC0Bits};
  else
    return i32x16{0};
}

template <int QK>
struct SAccT {
  using type = f32x16;
};
template <>
struct SAccT<kQK_INT8> {
  using type = i32x16;
};

// One 32-key half b of the S^T tile for this wave's 32 queries: acc covers
// keys 32b + (8j + 4h + i) in lane (h, r), element 4j + i.
template <int D, int QK, bool C0>
__device__ __forceinline__ void qk_half(const uint8_t* sb, const i32x4* qf, int lane, int b,
                                        typename SAccT<QK>::type& acc) {
  constexpr int NC = D / 32;
  const i32x4* kl = reinterpret_cast<const i32x4*>(sb);
  if constexpr (QK == kQK_INT8) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kl[(b * NC + c) * 64 + lane], qf[c], c == 0 ? i8_start<C0>() : acc,
                                                  0, 0, 0);
  } else {
    acc = f32x16{0};
#pragma unroll
    for (int c = 0; c < NC; c += 2) {
      const i32x8 bq = {qf[c][0], qf[c][1], qf[c][2], qf[c][3], qf[c + 1][0], qf[c + 1][1], qf[c + 1][2], qf[c + 1][3]};
      const i32x4 a0 = kl[(b * NC + c) * 64 + lane], a1 = kl[(b * NC + c + 1) * 64 + lane];
      const i32x8 ka = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ka, bq, acc, 0, 0, 0, 0, 0, 0);
    }
  }
}

// Both 32-key halves of the next S^T as two interleaved MFMA chains.
template <int D, int QK, bool C0>
__device__ __forceinline__ void qk_both(const uint8_t* sb, const i32x4* qf, int lane, typename SAccT<QK>::type& a0,
                                        typename SAccT<QK>::type& a1) {
  constexpr int NC = D / 32;
  const i32x4* kl = reinterpret_cast<const i32x4*>(sb);
  if constexpr (QK == kQK_INT8) {
    // K fragments read two chunks ahead of their MFMAs: the chain waits for
    // one LDS latency, not one per MFMA
    i32x4 kf[2][NC];
    auto read = [&](int c) __attribute__((always_inline)) {
      kf[0][c] = kl[(0 * NC + c) * 64 + lane];
      kf[1][c] = kl[(1 * NC + c) * 64 + lane];
    };
    read(0);
    read(1);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      __builtin_amdgcn_sched_barrier(0);
      a0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[0][c], qf[c], c == 0 ? i8_start<C0>() : a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[1][c], qf[c], c == 0 ? i8_start<C0>() : a1, 0, 0, 0);
      if (c + 2 < NC) read(c + 2);
    }
  } else {
    qk_half<D, QK, C0>(sb, qf, lane, 0, a0);
    qk_half<D, QK, C0>(sb, qf, lane, 1, a1);
  }
}

// Per-row values for the O fragment: lane (h, r) holds rows 8j + 4h + i,
// element 4j + i.  Lanes h = 0 publish their row's value in the wave's
// 32-float exchange; every lane then reads four broadcast float4s.
// The exchange passes values between lanes, which a single-lane view of the
// program does not see: wavefront-scope fences around it keep the compiler
// from reusing an earlier call's reads in a later call.
__device__ __forceinline__ void rows_of(float* xrow, float v, int h, int r, float out[16]) {
  if (h == 0) xrow[r] = v;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const f32x4* x4 = reinterpret_cast<const f32x4*>(xrow);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x4 q = x4[2 * j + h];
#pragma unroll
    for (int i = 0; i < 4; ++i) out[4 * j + i] = q[i];
  }
}

// Scores of the 32-key half b of the tile in stage sb from its S^T
// accumulators s: u = acc * kd (log2 units before the query scale), with kd
// the per-key K scale (token granularity, from the stage) or the tile's block
// scale kd_blk.  Keys at or past kvalid (the keys of the tile below N) get
// -inf: only the ragged last tile tests.  With masked set (DOC), the
// per-token document-id visibility: key visible iff doc[key] >= 0 and
// (doc[q] == doc[key] or doc[q] < 0).
template <int D, int QK, int PV, int GRAN, bool DOC, bool C0>
__device__ __forceinline__ void half_scores(const uint8_t* sb, const typename SAccT<QK>::type& s, int b, int h,
                                            float kd_blk, int kvalid, bool masked, int dq, float (&u)[16]) {
  using St = Stage<D, PV>;
  const f32x4* kdl = reinterpret_cast<const f32x4*>(sb + St::offKd);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f32x4 kd4;
    if constexpr (GRAN == kGRAN_TOKEN)
      kd4 = kdl[8 * b + 2 * j + h];
    else
      kd4 = f32x4{kd_blk, kd_blk, kd_blk, kd_blk};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (QK == kQK_INT8 && C0)
        u[4 * j + i] = (__int_as_float(s[4 * j + i]) - kC0) * kd4[i];  // acc * kd * 2^-26
      else if constexpr (QK == kQK_INT8)
        u[4 * j + i] = (float)s[4 * j + i] * kd4[i];
      else
        u[4 * j + i] = s[4 * j + i] * kd4[i];
    }
  }
  if (kvalid < 64) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (32 * b + 8 * j + 4 * h + i >= kvalid) u[4 * j + i] = -INFINITY;
  }
  if constexpr (DOC) {
    if (masked) {
      const int4* dkl = reinterpret_cast<const int4*>(sb + St::offDoc);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int4 dk4 = dkl[8 * b + 2 * j + h];
        const int dk[4] = {dk4.x, dk4.y, dk4.z, dk4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!(dk[i] >= 0 && (dq == dk[i] || dq < 0))) u[4 * j + i] = -INFINITY;
      }
    }
  }
}

// Row max of the tile's 32 scores per lane (max3 tree, then across the two
// lane halves) in log2 units, and the lazy frame move: the reference point
// m_ref moves to the block max bm when bm exceeds it by more than kTau, and
// O and l are rescaled then (branch-free values, the O rescale only when some
// row of the wave moves).  Returns bm (-inf for a row that sees no key).
// row_max_frame decides the move and rescales l; it sets any_move when some
// row of the wave moved, and the caller rescales O by alpha (frame_move_o),
// at once (row_max_move) or before the next product is added to O.
__device__ __forceinline__ float row_max_frame(float (&u)[2][16], float wt, float& m_ref, float& l_acc, float& alpha,
                                               bool& any_move) {
  constexpr float kTau = 8.0f;
  float mx;
  {
    auto max3 = [](float a, float b, float c) { return __builtin_fmaxf(__builtin_fmaxf(a, b), c); };
    const float* w = &u[0][0];
    float l1[12];
#pragma unroll
    for (int k = 0; k < 10; ++k) l1[k] = max3(w[3 * k], w[3 * k + 1], w[3 * k + 2]);
    l1[10] = w[30];
    l1[11] = w[31];
    const float l2a = max3(l1[0], l1[1], l1[2]), l2b = max3(l1[3], l1[4], l1[5]);
    const float l2c = max3(l1[6], l1[7], l1[8]), l2d = max3(l1[9], l1[10], l1[11]);
    mx = __builtin_fmaxf(max3(l2a, l2b, l2c), l2d);
  }
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
  }
  const float bm = mx * wt;  // -inf if nothing visible in this row
  const bool row_live = bm > -INFINITY;
  const bool move = row_live && !(bm <= m_ref + kTau);
  alpha = move ? __builtin_amdgcn_exp2f(m_ref - bm) : 1.0f;  // 0 when m_ref = -inf
  m_ref = move ? bm : m_ref;
  l_acc *= alpha;
  any_move = __any(move);
  return bm;
}

// O *= alpha of its row (the frame move of row_max_frame).
template <int D>
__device__ __forceinline__ void frame_move_o(f32x16* o, float* xrow, float alpha, int h, int r) {
  constexpr int NC = D / 32;
  float arow[16];
  rows_of(xrow, alpha, h, r, arow);
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[c][e] *= arow[e];
}

template <int D>
__device__ __forceinline__ float row_max_move(float (&u)[2][16], float wt, float& m_ref, float& l_acc, f32x16* o,
                                              float* xrow, int h, int r) {
  float alpha;
  bool any_move;
  const float bm = row_max_frame(u, wt, m_ref, l_acc, alpha, any_move);
  if (any_move) frame_move_o<D>(o, xrow, alpha, h, r);
  return bm;
}

// The exp / pack part of the fp8 softmax for fp8 QK (after the frame decision
// for block max bm: P codes into pa, the row factor into rsc, the row sum into
// l), with the next tile's S^T (K of stage sb_next) issued among its vector
// work: the MFMAs of the two halves (their chains alternate) in four groups,
// each followed by the exp / pack work of 8 of the lane's 32 scores, with
// scheduling fences between the groups, so the wave keeps issuing vector
// instructions while its matrix core forms the next S^T.  K fragments are
// read two MFMAs ahead.
template <int D>
__device__ __forceinline__ void softmax_fp8_exp_qk(const float (&u)[2][16], float wt, float bm, float m_ref,
                                                   float& l_acc, i32x8& pa, float& rsc, const uint8_t* sb_next,
                                                   const i32x4* qf, int lane, f32x16& a0, f32x16& a1) {
  constexpr int NC = D / 32;
  constexpr int kM = NC;  // MFMA i: half i & 1, channels 64 (i >> 1) .. + 63
  const i32x4* kl = reinterpret_cast<const i32x4*>(sb_next);
  i32x4 kf[kM][2];
  auto read = [&](int i) __attribute__((always_inline)) {
    const int b = i & 1, c = (i >> 1) * 2;
    kf[i][0] = kl[(b * NC + c) * 64 + lane];
    kf[i][1] = kl[(b * NC + c + 1) * 64 + lane];
  };
  auto mfma = [&](int i) __attribute__((always_inline)) {
    const int b = i & 1, c = (i >> 1) * 2;
    f32x16& acc = b ? a1 : a0;
    const i32x8 bq = {qf[c][0], qf[c][1], qf[c][2], qf[c][3], qf[c + 1][0], qf[c + 1][1], qf[c + 1][2], qf[c + 1][3]};
    const i32x8 ka = {kf[i][0][0], kf[i][0][1], kf[i][0][2], kf[i][0][3],
                      kf[i][1][0], kf[i][1][1], kf[i][1][2], kf[i][1][3]};
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ka, bq, i < 2 ? f32x16{0} : acc, 0, 0, 0, 0, 0, 0);
  };
  read(0);
  if (kM > 1) read(1);
  const bool row_live = bm > -INFINITY;
  rsc = row_live ? __builtin_amdgcn_exp2f(bm - m_ref) * (1.0f / kFp8Max) : 0.0f;
  const float bias = row_live ? (kLog2Fp8Max - bm) : 0.0f;  // masked u are -inf: e = 0
  float es[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = g * kM / 4; i < (g + 1) * kM / 4; ++i) {
      mfma(i);
      if (i + 2 < kM) read(i + 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    // scores of half g >> 1, rows 8j + 4h + i for j = 2 (g & 1) .. + 1
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int b = g >> 1, j = 2 * (g & 1) + jj;
      float e4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e4[i] = __builtin_amdgcn_exp2f(fmaf(u[b][4 * j + i], wt, bias));
        es[i] += e4[i];
      }
      pa[4 * b + j] = (int)pack_fp8x4(e4[0], e4[1], e4[2], e4[3]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  l_acc = fmaf(rsc, (es[0] + es[1]) + (es[2] + es[3]), l_acc);
}

// The exp / pack part of the fp8 softmax after the frame decision for block
// max bm: P codes into pa, the row factor into rsc, the row sum into l.
__device__ __forceinline__ void softmax_fp8_exp(const float (&u)[2][16], float wt, float bm, float m_ref,
                                                float& l_acc, i32x8& pa, float& rsc) {
  const bool row_live = bm > -INFINITY;
  rsc = row_live ? __builtin_amdgcn_exp2f(bm - m_ref) * (1.0f / kFp8Max) : 0.0f;
  const float bias = row_live ? (kLog2Fp8Max - bm) : 0.0f;  // masked u are -inf: e = 0
  float es[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float e4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e4[i] = __builtin_amdgcn_exp2f(fmaf(u[b][4 * j + i], wt, bias));
        es[i] += e4[i];
      }
      pa[4 * b + j] = (int)pack_fp8x4(e4[0], e4[1], e4[2], e4[3]);
    }
  l_acc = fmaf(rsc, (es[0] + es[1]) + (es[2] + es[3]), l_acc);
}

template <int D>
__device__ __forceinline__ void softmax_fp8(float (&u)[2][16], float wt, float& m_ref, float& l_acc, f32x16* o,
                                            float* xrow, int h, int r, i32x8& pa, float& rsc) {
  const float bm = row_max_move<D>(u, wt, m_ref, l_acc, o, xrow, h, r);
  softmax_fp8_exp(u, wt, bm, m_ref, l_acc, pa, rsc);
}

// fp8 P.V of one tile for the chunk pair (c2, c2 + 1): the block products
// p0, p1 (v_mfma_f32_32x32x64_f8f6f4, P codes pa against the V codes of stage
// sb) and their dequantization factors rsc[row] * vd[channel] in the O layout.
// The factors are rank-1 products made on the matrix cores:
// v_mfma_f32_32x32x1_2b_f32 forms two 32x32 outer products, block b from the
// lanes h = b, with A = rsc of query r (lane-local in the S^T layout) and B =
// the V scale of channel 32(c2 + b) + r; each product is one correctly
// rounded fp32 multiply, as on the vector ALU, and no lane exchange is needed.
// The stage operands of one chunk pair's fp8 P.V: the V fragments of chunks
// c2 and c2 + 1 and the V scale this lane feeds the factor MFMA.
struct PvFrags {
  i32x4 v[4];
  float vd;
};

template <int D>
__device__ __forceinline__ PvFrags pv_load(const uint8_t* sb, int lane, int c2) {
  using St = Stage<D, kPV_FP8>;
  const int h = lane >> 5, r = lane & 31;
  const i32x4* vl = reinterpret_cast<const i32x4*>(sb + St::offV);
  const float* vdl = reinterpret_cast<const float*>(sb + St::offVd);
  PvFrags f;
#pragma unroll
  for (int i = 0; i < 4; ++i) f.v[i] = vl[(c2 * 2 + i) * 64 + lane];
  f.vd = vdl[32 * (c2 + h) + r];
  return f;
}

template <int D>
__device__ __forceinline__ void pv_issue_f(const PvFrags& f, const i32x8& pa, float rsc, f32x16& p0, f32x16& p1,
                                           f32x32& rv) {
  rv = __builtin_amdgcn_mfma_f32_32x32x1f32(rsc, f.vd, f32x32{0}, 0, 0, 0);
  auto pv = [&](int i) {
    const i32x4 b0 = f.v[2 * i], b1 = f.v[2 * i + 1];
    const i32x8 bv = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(pa, bv, f32x16{0}, 0, 0, 0, 0, 0, 0);
  };
  p0 = pv(0);
  p1 = pv(1);
}

template <int D>
__device__ __forceinline__ void pv_issue(const uint8_t* sb, const i32x8& pa, float rsc, int lane, int c2, f32x16& p0,
                                         f32x16& p1, f32x32& rv) {
  pv_issue_f<D>(pv_load<D>(sb, lane, c2), pa, rsc, p0, p1, rv);
}

__device__ __forceinline__ void pv_accum(f32x16* o, int c2, const f32x16& p0, const f32x16& p1, const f32x32& rv) {
#pragma unroll
  for (int e = 0; e < 16; ++e) o[c2][e] = fmaf(p0[e], rv[e], o[c2][e]);
#pragma unroll
  for (int e = 0; e < 16; ++e) o[c2 + 1][e] = fmaf(p1[e], rv[16 + e], o[c2 + 1][e]);
}

// bf16 P of the tile: 2^(s - m_ref) <= 2^kTau after the frame decision, row
// sums into l.  O is not touched: the caller applies the move (alpha, when
// the result is true) to O before it adds this tile's product.
__device__ __forceinline__ bool softmax_bf16(float (&u)[2][16], float wt, float& m_ref, float& l_acc,
                                             bf16x8 (&pa)[2][2], float& alpha) {
  bool any_move;
  const float bm = row_max_frame(u, wt, m_ref, l_acc, alpha, any_move);
  const float bias = bm > -INFINITY ? -m_ref : 0.0f;  // masked u are -inf: p = 0
  float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pr = __builtin_amdgcn_exp2f(fmaf(u[b][e], wt, bias));
      ls[e & 3] += pr;
      pa[b][e >> 3][e & 7] = (__bf16)pr;
    }
  l_acc += (ls[0] + ls[1]) + (ls[2] + ls[3]);
  return any_move;
}

// bf16 P.V of the channel chunks c0 and c0 + 1 of one tile, accumulated
// straight into O: 8 v_mfma_f32_32x32x16_bf16 as two interleaved chains, the
// V fragments (fragment (c * 2 + b) * 2 + tt of the stage) read first.
template <int D>
__device__ __forceinline__ void pv_bf16_pair(const uint8_t* sb, const bf16x8 (&pa)[2][2], int lane, int c0,
                                             f32x16* o) {
  using St = Stage<D, kPV_BF16>;
  const bf16x8* vl = reinterpret_cast<const bf16x8*>(sb + St::offV);
  bf16x8 vf[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) vf[j] = vl[((c0 + (j & 1)) * 4 + (j >> 1)) * 64 + lane];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = c0 + (j & 1), k = j >> 1;
    o[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[k >> 1][k & 1], vf[j], o[c], 0, 0, 0);
  }
}

// The per-tile work of one wave in the general loop, as straight-line code
// for the scheduler: scores of tile t from s0/s1, the next tile's S^T into
// s0/s1 (both halves issued first, as two interleaved MFMA chains, so the
// matrix cores overlap this tile's vector work), online softmax, then P.V:
// bf16 accumulated straight into O, or fp8 dequantized into O right away.
// MASKED selects the per-token document-id visibility test.
template <int D, int QK, int PV, int GRAN, int MASK, bool MASKED>
__device__ __forceinline__ void tile_body(const uint8_t* sb, const uint8_t* sb_next, const i32x4* qf, int lane,
                                          typename SAccT<QK>::type& s0, typename SAccT<QK>::type& s1, f32x16* o,
                                          float& m_ref, float& l_acc, float wt, float* xrow, int dq, float kd_blk,
                                          int kvalid) {
  using St = Stage<D, PV>;
  constexpr int NC = D / 32;
  const int h = lane >> 5, r = lane & 31;
  constexpr bool C0 = (MASK & 2) != 0;  // the int8 chains' start (i8_start)
  float u[2][16];
  half_scores<D, QK, PV, GRAN, MASKED, C0>(sb, s0, 0, h, kd_blk, kvalid, true, dq, u[0]);
  half_scores<D, QK, PV, GRAN, MASKED, C0>(sb, s1, 1, h, kd_blk, kvalid, true, dq, u[1]);
  qk_both<D, QK, C0>(sb_next, qf, lane, s0, s1);
  if constexpr (PV == kPV_FP8) {
    i32x8 pa;
    float rsc;
    softmax_fp8<D>(u, wt, m_ref, l_acc, o, xrow, h, r, pa, rsc);
#pragma unroll
    for (int c2 = 0; c2 < NC; c2 += 2) {
      f32x16 p0, p1;
      f32x32 rv;
      pv_issue<D>(sb, pa, rsc, lane, c2, p0, p1, rv);
      pv_accum(o, c2, p0, p1, rv);
    }
    return;
  }
  // bf16 P = 2^(s - m_ref) <= 2^kTau, accumulated straight into O
  bf16x8 pa[2][2];
  float alpha;
  if (softmax_bf16(u, wt, m_ref, l_acc, pa, alpha)) frame_move_o<D>(o, xrow, alpha, h, r);
  // V fragments read four MFMAs ahead of their use: the chain waits for one
  // LDS latency, not one per MFMA
  const bf16x8* vl = reinterpret_cast<const bf16x8*>(sb + St::offV);
  constexpr int kPV = NC * 4, kAhead = 4;
  bf16x8 vf[kPV];
#pragma unroll
  for (int i = 0; i < kAhead; ++i) vf[i] = vl[i * 64 + lane];
#pragma unroll
  for (int i = 0; i < kPV; ++i) {
    __builtin_amdgcn_sched_barrier(0);
    const int c = i >> 2, b = (i >> 1) & 1, tt = i & 1;  // fragment ((c * 2 + b) * 2 + tt) = i
    o[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[b][tt], vf[i], o[c], 0, 0, 0);
    if (i + kAhead < kPV) vf[i + kAhead] = vl[(i + kAhead) * 64 + lane];
  }
}

// Tiles [t_begin, t_end) of work item (bh, query tile qt) for this wave:
// leaves the wave's O, reference point and row-sum half in o / m_ref / l_acc
// (O and l in the frame of m_ref; all zero / -inf for a wave past N).
// Ends with a workgroup barrier, after which the stage ring may be reused.
// DUMP (per-token scales) also stores every S^T accumulator pair this loop
// consumes into p.s_dump, at the point where it is consumed.
template <int D, int QK, int PV, int GRAN, int MASK, bool DUMP = false>
__device__ __forceinline__ bool item_tiles(const AttnParams& p, uint8_t* smem, int bh, int qt, int t_begin,
                                           int t_end, f32x16* o, float& m_ref, float& l_acc,
                                           bool skip_listed = false) {
  bool listed = false;
  using St = Stage<D, PV>;
  using SM = Smem<D, PV>;
  using SAcc = typename SAccT<QK>::type;
  constexpr int NC = D / 32;  // 32-channel chunks
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, r = lane & 31;
  const int nq = (int)(p.np / kRowsPerWG);
  const int bidx = bh / p.h;
  const int64_t q0 = (int64_t)qt * kRowsPerWG + 32 * wave;  // first query row of this wave
  const bool wave_live = q0 < p.n;
  float* xrow = reinterpret_cast<float*>(smem + SM::offX) + 32 * wave;

  m_ref = -INFINITY;
  l_acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NC; ++j) o[j] = f32x16{0};

  // ---- per-wave query state ------------------------------------------------
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
  // the int8 chains' start (i8_start): from c0 with document ids
  constexpr bool kC0Start = (MASK & 2) != 0;
  // log2-domain multiplier of the (K-scaled) accumulators; int8 QK scores
  // started from c0 carry 2^-26, which the multiplier takes back exactly
  const float w = fmaxf(qd, 1e-30f) * (QK == kQK_INT8 && kC0Start ? kC0Scale : 1.0f);

  int dq = 0;
  int4 qsum = make_int4(0, 0, 0, 0), qsum128 = make_int4(0, 0, 0, 0);
  if (MASK & 2) {
    const int64_t qq = q0 + r;
    dq = qq < p.n ? p.doc[(int64_t)bidx * p.n + qq] : -1;
    // wave- and workgroup-uniform summaries: scalar loads into scalar registers
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    qsum = load_uniform(p.q_sum, (int64_t)bidx * (p.np / 32) + qt * 4 + wave_s);
    qsum128 = load_uniform(p.q_sum128, (int64_t)bidx * nq + qt);
  }

  const uint8_t* kg = p.kc + (int64_t)bh * p.np * D;
  const uint8_t* vg = p.vin + (int64_t)bh * p.np * D * (PV == kPV_FP8 ? 1 : 2);
  const int32_t* docb = (MASK & 2) ? p.doc + (int64_t)bidx * p.n : nullptr;

  // ---- tile schedule: active tiles in order ----------------------------------
  auto next_active = [&](int t) -> int {
    for (; t < t_end; ++t) {
      if (MASK & 1) {
        if (load_uniform_u8(p.tile_mask, (int64_t)bh * p.mask_stride_z + (int64_t)qt * p.mask_nkv + t) == 0) continue;
      }
      if (MASK & 2) {
        if (classify(qsum128, load_uniform(p.kv_sum, (int64_t)bidx * p.nt + t)) == 0) continue;
      }
      break;
    }
    return t;
  };

  // ---- loads: global -> LDS stage --------------------------------------------
  // The K and V parts in 64-chunk blocks spread over the four waves, the K and
  // V scales by lanes of wave 0, all as direct global -> LDS loads; the key
  // document ids (bounds-checked: -1 past N) through registers of threads
  // 48..63.  The caller waits for vmcnt(0) before the barrier that publishes
  // the stage.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  int4 pre_doc = make_int4(-1, -1, -1, -1);
  // buffer resources over this head's K and V operands and scales: the stage
  // copies take a scalar tile offset and a loop-invariant lane offset
  const __amdgpu_buffer_rsrc_t rs_k = raw_rsrc(kg, (uint32_t)(p.np * D));
  const __amdgpu_buffer_rsrc_t rs_v = raw_rsrc(vg, (uint32_t)(p.np / 64 * St::vBytes));
  const __amdgpu_buffer_rsrc_t rs_ks = raw_rsrc(p.ks + (int64_t)bh * p.np, (uint32_t)(p.np * 4));
  const __amdgpu_buffer_rsrc_t rs_vs =
      raw_rsrc(PV == kPV_FP8 ? p.vs + (int64_t)bh * (p.np / 64) * D : p.ks, (uint32_t)(p.np / 64 * D * 4));
  // document ids of the keys, copied like the scales (fp8 P.V).  The whole
  // offset goes in the vector operand, the part the buffer range check
  // covers (per dword for a 16-byte load), so ids past N read as 0 and no
  // byte past the caller's [B, N] array is fetched; no score sees those ids,
  // since keys past N are masked by count
  constexpr bool kDocDma = (MASK & 2) && PV == kPV_FP8;
  const __amdgpu_buffer_rsrc_t rs_doc =
      raw_rsrc(kDocDma ? static_cast<const void*>(docb) : static_cast<const void*>(p.ks), (uint32_t)(p.n * 4));
  auto load_k = [&](int tt, uint8_t* sbw) __attribute__((always_inline)) {
    dma_chunks_buf<St::cK, 4>(sbw, wave_u, lane, rs_k, tt * 64 * D);
  };
  // the rest of the stage: V, the scales, the document ids
  auto load_v = [&](int tt, uint8_t* sbw) __attribute__((always_inline)) {
    dma_chunks_buf<St::cV, 4>(sbw + St::offV, wave_u, lane, rs_v, tt * St::vBytes);
    if (wave_u == 0) {
      // K scales by lanes 0..15 (64 keys), V scales by lanes 16.. (D
      // channels); lane l lands at byte 16 l of the scale region
      if (GRAN == kGRAN_TOKEN && lane < 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_ks, sbw + St::offKd, 16, lane * 16, tt * 256, 0, 0);
      if (PV == kPV_FP8 && lane >= 16 && lane < 16 + D / 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_vs, sbw + St::offKd, 16, (lane - 16) * 16, tt * D * 4, 0, 0);
    }
    if (kDocDma && wave_u == 1 && lane < 16)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_doc, sbw + St::offDoc, 16, tt * 256 + lane * 16, 0, 0, 0);
    if (!kDocDma && (MASK & 2) && tid >= 48 && tid < 64) {
      const int64_t base = (int64_t)tt * 64 + (tid - 48) * 4;
      pre_doc.x = base + 0 < p.n ? docb[base + 0] : -1;
      pre_doc.y = base + 1 < p.n ? docb[base + 1] : -1;
      pre_doc.z = base + 2 < p.n ? docb[base + 2] : -1;
      pre_doc.w = base + 3 < p.n ? docb[base + 3] : -1;
    }
  };
  auto load_tile = [&](int tt, uint8_t* sbw) __attribute__((always_inline)) {
    load_k(tt, sbw);
    load_v(tt, sbw);
  };
  auto store_doc = [&](uint8_t* sbw) __attribute__((always_inline)) {
    if (!kDocDma && (MASK & 2) && tid >= 48 && tid < 64) reinterpret_cast<int4*>(sbw + St::offDoc)[tid - 48] = pre_doc;
  };
  auto kd_block = [&](int tt) -> float {
    return GRAN == kGRAN_TOKEN ? 0.0f : load_uniform(p.ks, (int64_t)bh * (p.np / 64) + tt);
  };
  auto keys_valid = [&](int tt) -> int { return p.n - (int64_t)tt * 64 < 64 ? (int)(p.n - (int64_t)tt * 64) : 64; };
  // the S^T accumulators of tile tt (keys 64 tt + 32 b + 8 j + 4 h + i of
  // query q0 + r) as the loop consumes them; only live waves call it, so
  // q0 + r < Np, and every key index is below 64 nt <= Np
  // (int32 for int8 QK, the bit patterns of the fp32 sums for fp8 QK)
  auto dump = [&](int tt, const SAcc& a0, const SAcc& a1) __attribute__((always_inline)) {
    if constexpr (DUMP) {
      int32_t* row = p.s_dump + ((int64_t)bh * p.np + q0 + r) * p.np + (int64_t)tt * 64 + 4 * h;
      auto word = [](auto x) -> int32_t {
        if constexpr (QK == kQK_INT8) return kC0Start ? x - kC0Bits : x;  // the sum itself
        else return __float_as_int(x);
      };
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          row[8 * j + i] = word(a0[4 * j + i]);
          row[32 + 8 * j + i] = word(a1[4 * j + i]);
        }
    }
  };

  constexpr bool DOC = (MASK & 2) != 0;
  // the software-pipelined loop: every fp8 P.V variant, and bf16 P.V without
  // document ids
  constexpr bool kFast = PV == kPV_FP8 || !DOC;
  // bf16 P.V on the pipelined loop keeps three stages: a tile's K part is
  // loaded two tiles ahead and its V part (with the scales) one tile ahead,
  // so the K of tile i+2 goes into the stage whose V (tile i-1) the pending
  // product still reads
  constexpr bool kSplit = kFast && PV == kPV_BF16;
  // Document ids: the item's scheduled tiles lie in [range.x, range.z), and
  // with fp8 P.V the tiles before prefix_end (one past the last that some
  // live wave does not see whole, from doc_prefix_kernel) go through the
  // general tile body with its per-element visibility test; the pipelined
  // loop computes every scheduled tile in every live wave with no test.
  int prefix_end = t_begin;
  if constexpr (DOC) {
    const int4 range = load_uniform(p.doc_range, (int64_t)bidx * nq + qt);
    // a listed split query tile belongs to one of the first workgroups
    // (doc_prefix_kernel): here it runs no tile and the caller stores
    // nothing.  No branch precedes the item's other loads, so they stay
    // beside the range's.
    listed = skip_listed && range.w != 0;
    t_begin = listed ? t_end : t_begin;
    t_begin = max(t_begin, range.x);
    t_end = min(t_end, range.z);
    if constexpr (kFast) prefix_end = range.y;
  }
  // ---- prologue: tiles 0 and 1 of the schedule in stages 0 and 1 --------------
  int t = next_active(t_begin);
  int t1 = t < t_end ? next_active(t + 1) : t_end;
  int t2 = t1 < t_end ? next_active(t1 + 1) : t_end;
  if (t < t_end) {
    load_tile(t, smem);
    store_doc(smem);
  }
  if (t1 < t_end) {
    if constexpr (kSplit) {
      load_k(t1, smem + St::bytes);
    } else {
      load_tile(t1, smem + St::bytes);
      store_doc(smem + St::bytes);
    }
  }
  wait_vmem();
  __syncthreads();
  SAcc s0, s1;  // S^T of the tile about to be consumed
  if (t < t_end && wave_live) {
    qk_both<D, QK, kC0Start>(smem, qf, lane, s0, s1);
  }

  // one tile of the general loop: tile t2 into a stage no wave reads any more
  // (the last barrier ended every read of it), tile t through tile_body with
  // this wave's visibility class, the next tile's S^T, publish, advance
  constexpr int kSt = SM::kStages;
  auto general_step = [&](int& stage) __attribute__((always_inline)) {
    const uint8_t* sb = smem + stage * St::bytes;
    const int stage1 = stage + 1 == kSt ? 0 : stage + 1;
    const int stage2 = stage1 + 1 == kSt ? 0 : stage1 + 1;
    // tile t2 into a stage no wave reads any more (the last barrier ended
    // every read of it)
    if (t2 < t_end) load_tile(t2, smem + stage2 * St::bytes);
    const float kdb = kd_block(t);
    const int kvalid = keys_valid(t);

    int cls = wave_live ? 1 : 0;
    if ((MASK & 2) && cls) cls = classify(qsum, load_uniform(p.kv_sum, (int64_t)bidx * p.nt + t));
    // the last tile recomputes its own S^T in place of a next tile's (unused)
    const uint8_t* sb_next = t1 < t_end ? smem + stage1 * St::bytes : sb;
    if (cls != 0) dump(t, s0, s1);
    if (cls == 2)
      tile_body<D, QK, PV, GRAN, MASK, true>(sb, sb_next, qf, lane, s0, s1, o, m_ref, l_acc, w, xrow, dq, kdb,
                                             kvalid);
    else if (cls == 1)
      tile_body<D, QK, PV, GRAN, MASK, false>(sb, sb_next, qf, lane, s0, s1, o, m_ref, l_acc, w, xrow, dq, kdb,
                                              kvalid);
    else if (wave_live && t1 < t_end)
      qk_both<D, QK, kC0Start>(sb_next, qf, lane, s0, s1);

    // ---- publish tile t2 ---------------------------------------------------------
    if (t2 < t_end) store_doc(smem + stage2 * St::bytes);
    wait_vmem();
    __syncthreads();
    stage = stage1;
    t = t1;
    t1 = t2;
    t2 = t2 < t_end ? next_active(t2 + 1) : t_end;
  };
  if constexpr (kFast) {
    // ---- every scheduled tile is computed by every live wave, so the product
    // of tile i-1 is always pending in iteration i.  The first and the last
    // tile are peeled off the loop, which leaves its body one straight basic
    // block for the scheduler: the pending P.V in two chunk-pair halves, each
    // under half of this tile's score conversion, then the next tile's S^T
    // under this tile's softmax.  fp8: the pending product's MFMAs and their
    // dequantization into O; bf16: its MFMAs accumulate into O, after the
    // frame move the previous softmax decided (deferred to here, so the
    // softmax never waits for the product in flight).  With document ids
    // (fp8) the tiles before prefix_end, which some live wave does not see
    // whole, go through the general body first; every later scheduled tile
    // is seen whole by every live wave.
    constexpr int NP = NC / 2;
    int stage = 0;
    if constexpr (DOC) {
      while (t < t_end && t < prefix_end) general_step(stage);
    }
    auto sp = [&](int s_) { return smem + s_ * St::bytes; };
    auto next_stage = [&](int s_, int k_) { return (s_ + k_) % kSt; };
    auto advance = [&]() __attribute__((always_inline)) {
      stage = next_stage(stage, 1);
      t = t1;
      t1 = t2;
      t2 = t2 < t_end ? next_active(t2 + 1) : t_end;
    };
    auto issue_loads = [&]() __attribute__((always_inline)) {
      if constexpr (kSplit) {
        if (t2 < t_end) load_k(t2, sp(next_stage(stage, 2)));
        if (t1 < t_end) load_v(t1, sp(next_stage(stage, 1)));
      } else {
        if (t2 < t_end) load_tile(t2, sp(next_stage(stage, 2)));
      }
    };
    auto publish = [&]() __attribute__((always_inline)) {
      if (t2 < t_end) store_doc(sp(next_stage(stage, 2)));
      wait_vmem();
      __syncthreads();
    };
    if (!wave_live) {
      // rows past N: the same loads and barriers, nothing computed
      while (t < t_end) {
        issue_loads();
        publish();
        advance();
      }
      __syncthreads();
      return !listed;
    }
    const bool any = t < t_end;
#ifdef SAGE_PHASE_TIMING
    uint64_t ph_acc[kPhases] = {0, 0, 0, 0, 0, 0};
    uint64_t ph_last = __builtin_amdgcn_s_memtime();
    const uint64_t ph_start = ph_last;
    int ph_n = 0;
#endif
    // the pending product: fp8 P codes and their row factor, or bf16 P and
    // the frame move that precedes its accumulation
    i32x8 pa_p = {0, 0, 0, 0, 0, 0, 0, 0};
    float rsc_p = 0.0f;
    bf16x8 pb_p[2][2];
    float alpha_p = 1.0f;
    bool move_p = false;
    int stage_p = 0;
    // fp8: the first chunk pair's stage operands of the pending product, read
    // in the iteration that forms its P codes, before its softmax, whose
    // vector work covers their LDS latency (the barrier waits for every LDS
    // access in flight)
    PvFrags pf0;
    auto prefetch_pending = [&]() __attribute__((always_inline)) {
      if constexpr (PV == kPV_FP8) pf0 = pv_load<D>(sp(stage), lane, 0);  // the tile about to become pending
    };
    float u[2][16];
    auto softmax_p = [&]() __attribute__((always_inline)) {
      if constexpr (PV == kPV_FP8)
        softmax_fp8<D>(u, w, m_ref, l_acc, o, xrow, h, r, pa_p, rsc_p);
      else
        move_p = softmax_bf16(u, w, m_ref, l_acc, pb_p, alpha_p);
    };
    // the pending product, chunk pair c2 (its frame move first, for bf16)
    auto pending_pair = [&](const uint8_t* sbp, int c2) __attribute__((always_inline)) {
      if constexpr (PV == kPV_FP8) {
        f32x16 p0, p1;
        f32x32 rv;
        pv_issue<D>(sbp, pa_p, rsc_p, lane, c2, p0, p1, rv);
        pv_accum(o, c2, p0, p1, rv);
      } else {
        pv_bf16_pair<D>(sbp, pb_p, lane, c2, o);
      }
    };
    auto pending_move = [&]() __attribute__((always_inline)) {
      if constexpr (PV == kPV_BF16) {
        if (move_p) frame_move_o<D>(o, xrow, alpha_p, h, r);
      }
    };
    if (t < t_end) {  // first tile: nothing pending
      issue_loads();
      dump(t, s0, s1);
      const float kdb = kd_block(t);
      const int kvalid = keys_valid(t);
      half_scores<D, QK, PV, GRAN, false, kC0Start>(sp(stage), s0, 0, h, kdb, kvalid, false, dq, u[0]);
      half_scores<D, QK, PV, GRAN, false, kC0Start>(sp(stage), s1, 1, h, kdb, kvalid, false, dq, u[1]);
      if (t1 < t_end) qk_both<D, QK, kC0Start>(sp(next_stage(stage, 1)), qf, lane, s0, s1);
      prefetch_pending();
      softmax_p();
      stage_p = stage;
      publish();
      advance();
    }
    // one iteration for a whole tile t with a successor
    auto iteration = [&]() __attribute__((always_inline)) {
      SAGE_PHASE(0);  // loop overhead since the last iteration's end
      issue_loads();
      const uint8_t* sb = sp(stage);
      const uint8_t* sbp = sp(stage_p);
      const float kdb = kd_block(t);
      dump(t, s0, s1);
      auto scores = [&](int b_, float (&u_)[16]) __attribute__((always_inline)) {
        half_scores<D, QK, PV, GRAN, false, kC0Start>(sb, b_ ? s1 : s0, b_, h, kdb, 64, false, dq, u_);
      };
      pending_move();
      if constexpr (PV == kPV_FP8) {
        f32x16 p0, p1;
        f32x32 rv;
        pv_issue_f<D>(pf0, pa_p, rsc_p, p0, p1, rv);
        scores(0, u[0]);
        if constexpr (NP == 1) scores(1, u[1]);
        pv_accum(o, 0, p0, p1, rv);
        if constexpr (NP == 2) {
          // fp8 QK: the second pair's products and factors only once the
          // first pair's are consumed (with the next S^T formed later, both
          // at once would not fit the registers)
          if constexpr (QK == kQK_FP8) __builtin_amdgcn_sched_barrier(0);
          pv_issue<D>(sbp, pa_p, rsc_p, lane, 2, p0, p1, rv);
          scores(1, u[1]);
          pv_accum(o, 2, p0, p1, rv);
        }
      } else {
        // bf16: the first chunk pair's products under the score conversion
        // (int8 QK, whose conversion is longer), the rest under the softmax
        if constexpr (QK == kQK_INT8) pv_bf16_pair<D>(sbp, pb_p, lane, 0, o);
        scores(0, u[0]);
        scores(1, u[1]);
      }
      if constexpr (PV == kPV_FP8 && QK == kQK_FP8 && D == 128) {
        // fp8 QK, D = 128: the frame decision ends a scheduling region (its
        // rare O rescale is a branch); the next tile's S^T goes after it,
        // among the exp / pack work of this tile (A/B at 1x30x4416x128
        // fp8/fp8: 234.7 -> 230.7 us and 240.3 -> 235.7 us; with int8 QK the
        // same order measured 247.7 -> 250.8 us: the other wave of the SIMD
        // already covers the QK^T burst)
        prefetch_pending();
        const float bm = row_max_move<D>(u, w, m_ref, l_acc, o, xrow, h, r);
        softmax_fp8_exp_qk<D>(u, w, bm, m_ref, l_acc, pa_p, rsc_p, sp(next_stage(stage, 1)), qf, lane, s0, s1);
      } else {
        SAGE_PHASE(1);  // the pending product and this tile's score conversion
        qk_both<D, QK, kC0Start>(sp(next_stage(stage, 1)), qf, lane, s0, s1);
        if constexpr (PV == kPV_BF16) {
          if constexpr (QK != kQK_INT8) pv_bf16_pair<D>(sbp, pb_p, lane, 0, o);
          if constexpr (NP == 2) pv_bf16_pair<D>(sbp, pb_p, lane, 2, o);
        }
        SAGE_PHASE(2);  // the next tile's QK^T issue
        prefetch_pending();
        if constexpr (PV == kPV_FP8) {
          const float bm = row_max_move<D>(u, w, m_ref, l_acc, o, xrow, h, r);
          SAGE_PHASE(3);  // row max and frame decision
          softmax_fp8_exp(u, w, bm, m_ref, l_acc, pa_p, rsc_p);
        } else {
          softmax_p();
        }
        SAGE_PHASE(4);  // exp, row sums, P packing
      }
      stage_p = stage;
      publish();
      SAGE_PHASE(5);  // stage loads complete, workgroup barrier
      advance();
#ifdef SAGE_PHASE_TIMING
      ++ph_n;
#endif
    };
    // the pending product, one chunk pair's products in flight at a time
    auto flush = [&]() __attribute__((always_inline)) {
      const uint8_t* sbp = sp(stage_p);
      pending_move();
#pragma unroll
      for (int c2 = 0; c2 < NC; c2 += 2) {
        pending_pair(sbp, c2);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    while (t1 < t_end) iteration();
    if (t < t_end) {  // last tile: the pending product, then the tile with its P.V formed at once
      flush();
      const uint8_t* sb = sp(stage);
      dump(t, s0, s1);
      tile_body<D, QK, PV, GRAN, MASK, false>(sb, sb, qf, lane, s0, s1, o, m_ref, l_acc, w, xrow, dq, kd_block(t),
                                              keys_valid(t));
      publish();
      advance();
    } else if (any) {  // the single tile was also the first: its product is pending
      flush();
    }
#ifdef SAGE_PHASE_TIMING
    {
      const uint64_t ph_end = __builtin_amdgcn_s_memtime();
      const int slot = (int)blockIdx.x * 4 + wave;
      if (lane == 0 && slot < kPhaseSlots) {
#pragma unroll
        for (int k = 0; k < kPhases; ++k) sage_phase_buf[slot][k] += ph_acc[k];
        sage_phase_buf[slot][6] += (unsigned long long)ph_n;
        sage_phase_buf[slot][7] += ph_end - ph_start;
      }
    }
#endif
    __syncthreads();  // the ring is reused after
    return !listed;
  }
  if constexpr (!kFast) {
    int stage = 0;
    while (t < t_end) general_step(stage);
  }
  return !listed;
}

constexpr int kRawBufferWord3 = 0x00020000;  // word 3 of a raw (untyped) buffer resource, gfx9 family

// Normalize and store this wave's 32 rows of item (bh, qt) and their LSE.
// Stages bf16 rows in the stage ring (free after item_tiles' final barrier)
// for 16-byte stores.
template <int D, int PV>
__device__ __forceinline__ void store_rows_final(const AttnParams& p, uint8_t* smem, int bh, int qt, f32x16* o,
                                                 float m_ref, float l_acc) {
  using SM = Smem<D, PV>;
  constexpr int NC = D / 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int h = lane >> 5, r = lane & 31;
  const int64_t q0 = (int64_t)qt * kRowsPerWG + 32 * wave;
  if (q0 >= p.n) return;  // wave past N: nothing to store (no barrier inside)
  float* xrow = reinterpret_cast<float*>(smem + SM::offX) + 32 * wave;
  float l_tot;
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_acc), __float_as_uint(l_acc), false, false);
    l_tot = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  const bool empty = !(l_tot > 0.0f);
  if (h == 0 && q0 + r < p.n) p.lse[(int64_t)bh * p.n + q0 + r] = empty ? -INFINITY : (m_ref + log2f(l_tot));
  float srow[16];
  rows_of(xrow, empty ? 0.0f : 1.0f / l_tot, h, r, srow);
  uint16_t* ep = reinterpret_cast<uint16_t*>(smem) + wave * 32 * D;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = 8 * (e >> 2) + 4 * h + (e & 3);
#pragma unroll
    for (int c = 0; c < NC; ++c) ep[row * D + 32 * c + r] = f32_to_bf16_rne(o[c][e] * srow[e]);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
  __builtin_amdgcn_wave_barrier();
  // 16-byte stores through a buffer resource that ends after the last row
  // below N: the hardware drops the stores of rows past N.  The whole offset
  // goes in the vector operand, the part the range check covers.
  const int rows = p.n - q0 < 32 ? (int)(p.n - q0) : 32;
  const int bh_b = bh / p.h, bh_h = bh - bh_b * p.h;
  const int rs_bytes = (int)(p.out_rs * 2);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      p.out + bh_b * p.out_bs + bh_h * p.out_hs + q0 * p.out_rs, 0, (rows - 1) * rs_bytes + D * 2, kRawBufferWord3);
  constexpr int kRowsPerStore = 16 * 64 / (2 * D);  // rows one 64-lane 16-byte store covers
  const int voff = (lane * 16 / (2 * D)) * rs_bytes + (lane * 16) % (2 * D);
#pragma unroll
  for (int i = 0; i < 32 * D * 2 / (16 * 64); ++i) {
    const int off = (lane + 64 * i) * 16;  // row-major bytes: row off / (2D), column (off % 2D) / 2
    const i32x4 v = *reinterpret_cast<const i32x4*>(reinterpret_cast<const uint8_t*>(ep) + off);
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, voff + i * kRowsPerStore * rs_bytes, 0, 0);
  }
}

// Partial result of a piece of a split item: O in lane order (element e of
// chunk c of wave w at ((w*NC + c)*16 + e)*64 + lane), then m_ref and l_acc
// per lane.  Buffer stores: the per-element offsets are scalar constants.
template <int D>
__device__ __forceinline__ void store_partial(float* slot, const f32x16* o, float m_ref, float l_acc) {
  constexpr int NC = D / 32;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(slot, 0, (int)(kPartFloats<D> * 4), kRawBufferWord3);
  const int vo = (wave * NC * 16 * 64 + lane) * 4;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o[c][e]), rs, vo, (c * 16 + e) * 256, 0);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_ref), rs, tid * 4, 128 * D * 4, 0);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l_acc), rs, tid * 4, (128 * D + 256) * 4, 0);
}

// store_partial for the in-kernel merge: the same layout, written through to
// the device's coherence point by agent-scope relaxed atomic stores (sc1 on
// gfx950), so that the merging workgroup, on any XCD, reads it there once the
// writer's stores have completed.
template <int D>
__device__ __forceinline__ void store_partial_coherent(float* slot, const f32x16* o, float m_ref, float l_acc) {
  constexpr int NC = D / 32;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  uint32_t* s32 = reinterpret_cast<uint32_t*>(slot) + wave * NC * 16 * 64 + lane;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      __hip_atomic_store(s32 + (c * 16 + e) * 64, __float_as_uint(o[c][e]), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  uint32_t* tail = reinterpret_cast<uint32_t*>(slot) + 128 * D;
  __hip_atomic_store(tail + tid, __float_as_uint(m_ref), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(tail + 256 + tid, __float_as_uint(l_acc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// The merge of split item si by the workgroup of its last piece, with the
// operations of merge_split_kernel in the same order (so the same bits).  The
// partials are read by agent-scope relaxed atomic loads (sc1), issued after
// this piece's arrival was counted behind every other piece's, whose stores
// had completed before they counted.  fac: LDS [8][128] floats.
template <int D>
__device__ __forceinline__ void merge_pieces(const AttnParams& p, int64_t si, float* fac) {
  constexpr int NC = D / 32;
  constexpr int kMaxParts = 8;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, h = lane >> 5, r = lane & 31;
  const int parts = p.split_parts;
  const int nq = (int)(p.np / kRowsPerWG);
  const int64_t pos = p.n_whole + si;
  const int bh = (int)(pos / nq), qt = (int)(pos % nq);
  const int64_t q0 = (int64_t)qt * kRowsPerWG + 32 * w;
  const uint32_t* slots = reinterpret_cast<const uint32_t*>(p.part + si * parts * kPartFloats<D>);
  auto ld = [](const uint32_t* a) __attribute__((always_inline)) {
    return __uint_as_float(__hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  };
  if (lane < 32) {  // the factors of row `lane` of this wave's 32 rows
    const int row = lane;
    float m[kMaxParts], l[kMaxParts];
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q) {
      if (q < parts) {
        const uint32_t* sl = slots + q * kPartFloats<D> + 128 * D;
        m[q] = ld(sl + w * 64 + row);
        l[q] = ld(sl + 256 + w * 64 + row) + ld(sl + 256 + w * 64 + 32 + row);
        mx = fmaxf(mx, m[q]);
      }
    }
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q) {
      if (q < parts) {
        m[q] = m[q] > -INFINITY ? __builtin_amdgcn_exp2f(m[q] - mx) : 0.0f;
        tot = fmaf(m[q], l[q], tot);
      }
    }
    const bool empty = !(tot > 0.0f);
    const float inv = empty ? 0.0f : 1.0f / tot;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q)
      if (q < parts) fac[q * 128 + w * 32 + row] = m[q] * inv;
    if (q0 + row < p.n) p.lse[(int64_t)bh * p.n + q0 + row] = empty ? -INFINITY : (mx + log2f(tot));
  }
  __syncthreads();
  // lane (h, r) holds channel 32c + r of rows 8j + 4h + i (element 4j + i of chunk c)
  float acc[NC][16];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[c][e] = 0.0f;
#pragma unroll 1
  for (int q = 0; q < parts; ++q) {
    const uint32_t* s = slots + q * kPartFloats<D> + w * NC * 16 * 64 + lane;
    float x[NC][16];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) x[c][e] = ld(s + (c * 16 + e) * 64);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[c][e] = fmaf(fac[q * 128 + w * 32 + 8 * (e / 4) + 4 * h + (e % 4)], x[c][e], acc[c][e]);
  }
  const int bh_b = bh / p.h, bh_h = bh - bh_b * p.h;
  uint16_t* ob = p.out + bh_b * p.out_bs + bh_h * p.out_hs + q0 * p.out_rs + r;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = 8 * (e / 4) + 4 * h + (e % 4);
      if (q0 + row < p.n) ob[row * p.out_rs + 32 * c] = f32_to_bf16_rne(acc[c][e]);
    }
}

template <int D, int QK, int PV, int GRAN, int MASK, bool DUMP = false>
__global__ void __launch_bounds__(256, 2) attn_fwd_kernel(AttnParams p) {
  using SM = Smem<D, PV>;
  constexpr int NC = D / 32;
  __shared__ __attribute__((aligned(16))) uint8_t smem[SM::bytes];
  f32x16 o[NC];
  float m_ref, l_acc;
  const int nq = (int)(p.np / kRowsPerWG);

  int bh, qt;
  bool skip_listed = false;  // document ids: this workgroup leaves a listed split query tile to the first ones
  if constexpr (MASK == 0) {
    // Unmasked: items in head-major order.  Workgroups [0, n_whole) take whole
    // items, dealt to XCDs (workgroup i runs on XCD i % 8) in contiguous
    // ranges so that an XCD's resident workgroups share K/V tiles in its L2.
    // Later workgroups, dispatched last, take the pieces of the split items
    // and leave partials; the last piece of an item to arrive merges them
    // (merge_pieces), or merge_split_kernel does after the launch.
    const int64_t b = blockIdx.x;
    if (b >= p.n_whole) {
      const int64_t c = b - p.n_whole;
      const int64_t si = c / p.split_parts;
      const int64_t pos = p.n_whole + si;
      const int part = (int)(c % p.split_parts);
      bh = (int)(pos / nq);
      qt = (int)(pos % nq);
      const int t0 = (int)((int64_t)part * p.nt / p.split_parts);
      const int t1 = (int)((int64_t)(part + 1) * p.nt / p.split_parts);
      item_tiles<D, QK, PV, GRAN, 0, DUMP>(p, smem, bh, qt, t0, t1, o, m_ref, l_acc);
      if (p.merge_ctr == nullptr) {
        store_partial<D>(p.part + c * kPartFloats<D>, o, m_ref, l_acc);
        return;
      }
      store_partial_coherent<D>(p.part + c * kPartFloats<D>, o, m_ref, l_acc);
      wait_vmem();  // this piece's partial is at the coherence point before it counts
      __syncthreads();
      int* last = reinterpret_cast<int*>(smem);
      if (threadIdx.x == 0) *last = arrive_last(p.merge_ctr + si, p.merge_tag, p.split_parts) ? 1 : 0;
      __syncthreads();
      if (*last == 0) return;
      __syncthreads();  // every wave has read the decision before the factors reuse the LDS
      merge_pieces<D>(p, si, reinterpret_cast<float*>(smem));
      if (threadIdx.x == 0)
        __hip_atomic_store(p.merge_ctr + si, p.merge_tag << 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    const int x = (int)(b % 8);
    const int64_t local = b / 8, per = p.n_whole / 8, rem = p.n_whole % 8;
    const int64_t pos = x * per + (x < rem ? x : rem) + local;
    bh = (int)(pos / nq);
    qt = (int)(pos % nq);
  } else {
    const int id = blockIdx.x, total = gridDim.x;
    if constexpr ((MASK & 2) != 0) {
      // the first heavy_max * h workgroups: head id % h of listed split query
      // tile id / h (doc_prefix_kernel); the others run the usual order and
      // leave the listed items to them
      const int reserved = p.heavy_max * p.h;
      if (id < reserved) {
        const int e = id / p.h;
        if (e >= load_uniform(&p.heavy[0].x, 0)) return;
        const int it = load_uniform(&p.heavy[1 + e].x, 0);
        bh = (it / nq) * p.h + id % p.h;
        qt = it % nq;
      } else {
        item_of(id - reserved, total - reserved, p.bh, nq, p.light_last, bh, qt);
        skip_listed = true;
      }
    } else {
      item_of(id, total, p.bh, nq, p.light_last, bh, qt);
    }
  }
  if (!item_tiles<D, QK, PV, GRAN, MASK, DUMP>(p, smem, bh, qt, 0, p.nt, o, m_ref, l_acc, skip_listed)) return;
  store_rows_final<D, PV>(p, smem, bh, qt, o, m_ref, l_acc);
}

// Merges the pieces of the split items.  Block (split item, 32-row block w,
// row group j) covers rows 8j + 4h + i (i < 4) of the block, all channels.
// Row rho: M = max over pieces of m, L = sum 2^(m - M) * l,
// out = sum 2^(m - M) * O / L, lse = M + log2(L) (empty rows: 0 and -inf, as
// the attention kernel writes them).
template <int D>
__global__ void __launch_bounds__(256) merge_split_kernel(AttnParams p) {
  constexpr int NC = D / 32;
  constexpr int kMaxParts = 8;
  const int64_t si = blockIdx.x;
  const int w = (int)blockIdx.y, j = (int)blockIdx.z;
  const int parts = p.split_parts;
  const int nq = (int)(p.np / kRowsPerWG);
  const int64_t pos = p.n_whole + si;
  const int bh = (int)(pos / nq), qt = (int)(pos % nq);
  const int64_t q0 = (int64_t)qt * kRowsPerWG + 32 * w;
  if (q0 >= p.n) return;  // uniform over the block
  const float* slots = p.part + si * parts * kPartFloats<D>;
  __shared__ float fac[kMaxParts][8];  // rows 8j .. 8j + 7 of the block
  const int tid = threadIdx.x;
  // the partial O values first: they do not depend on the factors, so both
  // rounds of loads are in flight together
  const int c = tid >> 6, lane = tid & 63, h = lane >> 5, r = lane & 31;
  float x[kMaxParts][4];
  if (tid < NC * 64) {
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        x[q][i] = q < parts ? slots[q * kPartFloats<D> + ((w * NC + c) * 16 + 4 * j + i) * 64 + lane] : 0.0f;
  }
  if (tid < 8) {
    const int row = 8 * j + tid;
    float m[kMaxParts], l[kMaxParts];
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q) {
      if (q < parts) {
        const float* sl = slots + q * kPartFloats<D> + 128 * D;
        m[q] = sl[w * 64 + row];
        l[q] = sl[256 + w * 64 + row] + sl[256 + w * 64 + 32 + row];
        mx = fmaxf(mx, m[q]);
      }
    }
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q) {
      if (q < parts) {
        m[q] = m[q] > -INFINITY ? __builtin_amdgcn_exp2f(m[q] - mx) : 0.0f;
        tot = fmaf(m[q], l[q], tot);
      }
    }
    const bool empty = !(tot > 0.0f);
    const float inv = empty ? 0.0f : 1.0f / tot;
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q)
      if (q < parts) fac[q][tid] = m[q] * inv;
    if (q0 + row < p.n) p.lse[(int64_t)bh * p.n + q0 + row] = empty ? -INFINITY : (mx + log2f(tot));
  }
  __syncthreads();
  if (tid < NC * 64) {
    const int bh_b = bh / p.h, bh_h = bh - bh_b * p.h;
    uint16_t* ob = p.out + bh_b * p.out_bs + bh_h * p.out_hs + q0 * p.out_rs + 32 * c + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 8 * j + 4 * h + i;
      float acc = 0.0f;
#pragma unroll
      for (int q = 0; q < kMaxParts; ++q)
        if (q < parts) acc = fmaf(fac[q][4 * h + i], x[q][i], acc);
      if (q0 + row < p.n) ob[row * p.out_rs] = f32_to_bf16_rne(acc);
    }
  }
}

template <int D, int QK, int PV, int GRAN>
hipError_t launch_attn_g(int mask, const AttnParams& p, hipStream_t st) {
  const int64_t items = (int64_t)p.bh * (p.np / kRowsPerWG);
  const int64_t n_split = mask == 0 ? items - p.n_whole : 0;
  // with document ids the first heavy_max * h workgroups take the listed split query tiles
  const dim3 grid((unsigned)(mask == 0 ? p.n_whole + n_split * p.split_parts
                                       : items + ((mask & 2) ? (int64_t)p.heavy_max * p.h : 0)));
  // the accumulator dump exists for the per-token, unmasked kernels
  constexpr bool kDumpable = GRAN == kGRAN_TOKEN;
  if (p.s_dump != nullptr) {
    if (!kDumpable || mask != 0) return hipErrorInvalidValue;
    if constexpr (kDumpable) hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 0, true>), grid, dim3(256), 0, st, p);
  } else switch (mask) {
    case 0: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 0>), grid, dim3(256), 0, st, p); break;
    case 1: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 1>), grid, dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 2>), grid, dim3(256), 0, st, p); break;
    case 3: hipLaunchKernelGGL((attn_fwd_kernel<D, QK, PV, GRAN, 3>), grid, dim3(256), 0, st, p); break;
  }
  if (n_split > 0 && p.merge_ctr == nullptr)
    hipLaunchKernelGGL(merge_split_kernel<D>, dim3((unsigned)n_split, 4, 4), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <int D>
hipError_t launch_attn_d(int qk, int pv, int gran, int mask, const AttnParams& p, hipStream_t st) {
#define SAGE_A_CASE(QK_, PV_, G_) \
  if (qk == QK_ && pv == PV_ && gran == G_) return launch_attn_g<D, QK_, PV_, G_>(mask, p, st);
  SAGE_A_CASE(0, 0, 0) SAGE_A_CASE(0, 0, 1) SAGE_A_CASE(0, 1, 0) SAGE_A_CASE(0, 1, 1)
  SAGE_A_CASE(1, 0, 0) SAGE_A_CASE(1, 0, 1) SAGE_A_CASE(1, 1, 0) SAGE_A_CASE(1, 1, 1)
#undef SAGE_A_CASE
  return hipErrorInvalidValue;
}

// One wave per (batch, 128-row query tile): lanes scan the key tiles for the
// scheduled ones (some row of the query tile sees a key): the first and one
// past the last of them bound the item's tile loop (no scan of the unseen
// tiles before and after), and one past the last that some live 32-row wave
// of the tile does not see whole (classify != 1) ends its prefix: the
// pipelined fp8 loop of the attention kernel takes the tiles from there on,
// the tiles before go through the general tile body with its per-element
// visibility test.
// A query tile whose live waves see different key-tile ranges (a document
// boundary inside the tile) runs the union of those ranges through the
// general body and is the longest item of its launch; up to heavy_max such
// tiles per launch are listed (heavy[1 + e].x = b * nq + qt, heavy[0].x the
// count, by an atomic counter) and flagged (range.w = 1), and the attention
// kernel's first workgroups take them, so they do not end the launch.  The
// list's order depends on the atomics, not the results: each item is computed
// the same way whichever workgroup takes it.
__global__ void __launch_bounds__(256) doc_prefix_kernel(const int4* __restrict__ kv_sum,
                                                         const int4* __restrict__ q_sum,
                                                         const int4* __restrict__ q_sum128, int nb, int nq, int nt,
                                                         int4* __restrict__ range, int4* __restrict__ heavy,
                                                         int heavy_max) {
  const int lane = threadIdx.x & 63;
  const int64_t item = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;  // wave-uniform
  if (item >= (int64_t)nb * nq) return;
  const int b = (int)(item / nq), qt = (int)(item % nq);
  const int4 q128 = q_sum128[(int64_t)b * nq + qt];
  int4 qs[4];
#pragma unroll
  for (int w4 = 0; w4 < 4; ++w4) qs[w4] = q_sum[(int64_t)b * nq * 4 + qt * 4 + w4];
  int first = nt, last = -1, last_mixed = -1;
  int wf[4] = {nt, nt, nt, nt}, wl[4] = {-1, -1, -1, -1};  // per-wave first / last visible tile
  for (int t = lane; t < nt; t += 64) {
    const int4 ks = kv_sum[(int64_t)b * nt + t];
    if (classify(q128, ks) == 0) continue;  // not scheduled
    first = min(first, t);
    last = t;
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      if (qs[w4].z + qs[w4].w == 0) continue;  // wave past N
      const int c = classify(qs[w4], ks);
      if (c != 1) last_mixed = t;
      if (c != 0) {
        wf[w4] = min(wf[w4], t);
        wl[w4] = t;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    first = min(first, __shfl_xor(first, off));
    last = max(last, __shfl_xor(last, off));
    last_mixed = max(last_mixed, __shfl_xor(last_mixed, off));
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      wf[w4] = min(wf[w4], __shfl_xor(wf[w4], off));
      wl[w4] = max(wl[w4], __shfl_xor(wl[w4], off));
    }
  }
  bool split = false;
#pragma unroll
  for (int w4 = 1; w4 < 4; ++w4)
    if (qs[w4].z + qs[w4].w != 0 && (wf[w4] != wf[0] || wl[w4] != wl[0])) split = true;
  if (lane == 0) {
    int listed = 0;
    if (split && heavy != nullptr) {
      const int e = atomicAdd(reinterpret_cast<int*>(heavy), 1);
      if (e < heavy_max) {
        heavy[1 + e] = make_int4((int)item, 0, 0, 0);
        listed = 1;
      }
    }
    range[item] = make_int4(first, last_mixed + 1, last + 1, listed);
  }
}

hipError_t launch_doc_prefix(const int4* kv_sum, const int4* q_sum, const int4* q_sum128, int64_t n, int nb,
                             int4* range, int4* heavy, hipStream_t st) {
  const int nq = (int)(padded_len(n) / 128);
  const int nt = (int)((n + 63) / 64);
  const int64_t waves = (int64_t)nb * nq;
  hipLaunchKernelGGL(doc_prefix_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, kv_sum, q_sum, q_sum128,
                     nb, nq, nt, range, heavy, kHeavyMax);
  return hipGetLastError();
}

hipError_t launch_doc_summaries(const int32_t* doc, int64_t n, int nb, int4* kv_sum, int4* q_sum, int4* q_sum128,
                                int4* heavy, hipStream_t st) {
  const int64_t np = padded_len(n);
  const int nt = (int)((n + 63) / 64);
  const int64_t total = (int64_t)nb * (nt + np / 32 + np / 128);  // summaries, one wave each
  const int64_t blocks = (total + 3) / 4 < 8192 ? (total + 3) / 4 : 8192;
  hipLaunchKernelGGL(doc_summary_kernel, dim3((unsigned)blocks), dim3(256), 0, st, doc, n, np, nb, nt, kv_sum, q_sum,
                     q_sum128, heavy);
  return hipGetLastError();
}

hipError_t launch_attn(int qk, int pv, int gran, int mask, const AttnParams& p, int64_t d, int nb,
                       hipStream_t st) {
  if (mask & 2) {
    hipError_t e = launch_doc_summaries(p.doc, p.n, nb, const_cast<int4*>(p.kv_sum), const_cast<int4*>(p.q_sum),
                                        const_cast<int4*>(p.q_sum128), p.heavy, st);
    if (e != hipSuccess) return e;
    e = launch_doc_prefix(p.kv_sum, p.q_sum, p.q_sum128, p.n, nb, const_cast<int4*>(p.doc_range), p.heavy, st);
    if (e != hipSuccess) return e;
  }
  if (d == 128) return launch_attn_d<128>(qk, pv, gran, mask, p, st);
  if (d == 64) return launch_attn_d<64>(qk, pv, gran, mask, p, st);
  return hipErrorInvalidValue;
}

AttnWorkspace attn_workspace(int64_t b, int64_t h, int64_t n, int64_t d, bool masked) {
  const int64_t np = padded_len(n);
  const int64_t nt = (n + 63) / 64;
  const int64_t items = b * h * (np / kRowsPerWG);
  AttnWorkspace w;
  w.split = tail_split(items, nt);
  w.doc_off = 0;
  // summaries (int4), the per-query-tile scheduled ranges (int4), then the
  // list of split query tiles (a count and kHeavyMax entries)
  w.heavy_off = (size_t)(b * (nt + np / 32 + np / 128 + np / 128)) * sizeof(int4);
  w.part_off = (w.heavy_off + (size_t)(1 + kHeavyMax) * sizeof(int4) + 255) & ~(size_t)255;
  const int64_t split_items = !masked && w.split.parts > 1 ? items - w.split.whole : 0;
  const int64_t pieces = split_items * w.split.parts;
  // then one 8-byte arrival counter per split item (in-kernel merge)
  w.ctr_off = w.part_off + (size_t)pieces * (size_t)(128 * d + 512) * sizeof(float);
  w.bytes = w.ctr_off + (size_t)split_items * sizeof(uint64_t);
  return w;
}

size_t attn_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d, bool masked) {
  return attn_workspace(b, h, n, d, masked).bytes;
}

}  // namespace sage

#ifdef SAGE_PHASE_TIMING
// Measurement library only: copies min(count, slots * 8) words of the phase
// buffer to host memory, then clears the buffer when clear != 0.
extern "C" int sage_phase_read(unsigned long long* host, size_t count, int clear) {
  const size_t words = (size_t)sage::kPhaseSlots * 8;
  if (count > words) count = words;
  if (host && count &&
      hipMemcpyFromSymbol(host, HIP_SYMBOL(sage::sage_phase_buf), count * 8, 0, hipMemcpyDeviceToHost) != hipSuccess)
    return -1;
  if (clear) {
    void* dev = nullptr;
    if (hipGetSymbolAddress(&dev, HIP_SYMBOL(sage::sage_phase_buf)) != hipSuccess) return -1;
    if (hipMemset(dev, 0, words * 8) != hipSuccess) return -1;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
  }
  return 0;
}
#endif
