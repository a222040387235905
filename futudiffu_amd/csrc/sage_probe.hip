// Issue-cost and MFMA/VALU co-execution probes for gfx950.
//
// Measurement tooling behind `bench.py --isa-probe` (built into its own
// library, libsage_probe.so); nothing in the attention path uses it.  Every
// probe kernel times its own loop per wave with s_memtime (the shader clock)
// and stores one dword per thread and one cycle count per wave into buffers
// sized for its grid, so every access is in bounds.
//
// Issue costs: each wave runs kIssueIter iterations of 8 independent register
// chains of one instruction; ticks per wave-instruction at about one and two
// waves per SIMD (256 or 512 workgroups of 4 waves on 256 CUs).
// Co-execution: 512-thread workgroups, one per CU, so waves w and w + 4 share
// SIMD w; the modes give the two waves of a SIMD an MFMA stream, a VALU (FMA)
// stream, both in one wave, or idle.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kIssueIter = 256;

#define SAGE_PROBE_BODY8(INS)                           \
  asm volatile(INS : "+v"(a0) : "v"(k0), "v"(k1));      \
  asm volatile(INS : "+v"(a1) : "v"(k0), "v"(k1));      \
  asm volatile(INS : "+v"(a2) : "v"(k0), "v"(k1));      \
  asm volatile(INS : "+v"(a3) : "v"(k0), "v"(k1));      \
  asm volatile(INS : "+v"(a4) : "v"(k0), "v"(k1));      \
  asm volatile(INS : "+v"(a5) : "v"(k0), "v"(k1));      \
  asm volatile(INS : "+v"(a6) : "v"(k0), "v"(k1));      \
  asm volatile(INS : "+v"(a7) : "v"(k0), "v"(k1));

#define SAGE_PROBE_KERNEL(NAME, INS)                                                       \
  __global__ void __launch_bounds__(256) NAME(uint32_t* out, uint64_t* cyc, float seed) { \
    float k0 = seed * 0.5f, k1 = seed * 0.25f;                                            \
    float a0 = seed + threadIdx.x, a1 = a0 + 1, a2 = a0 + 2, a3 = a0 + 3;                 \
    float a4 = a0 + 4, a5 = a0 + 5, a6 = a0 + 6, a7 = a0 + 7;                             \
    const uint64_t t0 = __builtin_amdgcn_s_memtime();                                     \
    for (int i = 0; i < kIssueIter; ++i) {                                                \
      SAGE_PROBE_BODY8(INS)                                                               \
    }                                                                                     \
    const uint64_t t1 = __builtin_amdgcn_s_memtime();                                     \
    const int tid = blockIdx.x * blockDim.x + threadIdx.x;                               \
    out[tid] = __float_as_uint(a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7);                    \
    if ((threadIdx.x & 63) == 0) cyc[tid >> 6] = t1 - t0;                                 \
  }

SAGE_PROBE_KERNEL(p_fma, "v_fma_f32 %0, %0, %1, %2")
SAGE_PROBE_KERNEL(p_mul, "v_mul_f32 %0, %0, %1")
SAGE_PROBE_KERNEL(p_add, "v_add_f32 %0, %0, %1")
SAGE_PROBE_KERNEL(p_max3, "v_max3_f32 %0, %0, %1, %2")
SAGE_PROBE_KERNEL(p_cvt_i32, "v_cvt_f32_i32 %0, %0")
SAGE_PROBE_KERNEL(p_exp, "v_exp_f32 %0, %0")
SAGE_PROBE_KERNEL(p_cvt_fp8, "v_cvt_pk_fp8_f32 %0, %1, %2")
SAGE_PROBE_KERNEL(p_cvt_bf16, "v_cvt_pk_bf16_f32 %0, %1, %2")
SAGE_PROBE_KERNEL(p_pk_fma16, "v_pk_fma_f16 %0, %0, %1, %2")
SAGE_PROBE_KERNEL(p_dot2_bf16, "v_dot2_f32_bf16 %0, %1, %2, %0")

typedef void (*IssueFn)(uint32_t*, uint64_t*, float);
struct IssueProbe {
  const char* name;
  IssueFn fn;
};
const IssueProbe kIssue[] = {
    {"v_fma_f32", p_fma},           {"v_mul_f32", p_mul},         {"v_add_f32", p_add},
    {"v_max3_f32", p_max3},         {"v_cvt_f32_i32", p_cvt_i32}, {"v_exp_f32", p_exp},
    {"v_cvt_pk_fp8_f32", p_cvt_fp8}, {"v_cvt_pk_bf16_f32", p_cvt_bf16}, {"v_pk_fma_f16", p_pk_fma16},
    {"v_dot2_f32_bf16", p_dot2_bf16},
};
constexpr int kNumIssue = sizeof(kIssue) / sizeof(kIssue[0]);

// ---- co-execution ----------------------------------------------------------

constexpr int kCoIter = 64;

__device__ __forceinline__ void valu16(float (&x)[8], float k0, float k1) {
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[j]) : "v"(k0), "v"(k1));
}

// Roles of waves 0-3 (mode bits 0-1) and 4-7 (bits 2-3): 0 idle, 1 MFMA
// stream, 2 VALU stream, 3 both interleaved.  The MFMA stream is four pairs
// of MFMAs per iteration on two alternating accumulator chains (QK = 0:
// v_mfma_i32_32x32x32_i8, QK = 1: v_mfma_scale_f32_32x32x64_f8f6f4); the VALU
// stream VPM FMAs per MFMA pair.  Roles are wave-uniform scalars, so the role
// branches are scalar branches with no EXEC writes.
template <int QK, int VPM>
__global__ void __launch_bounds__(512) coexec_kernel(uint32_t* out, uint64_t* cyc, int mode) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int role = __builtin_amdgcn_readfirstlane(wave < 4 ? (mode & 3) : ((mode >> 2) & 3));
  const int lane = threadIdx.x & 63;
  const i32x4 a = {lane, lane + 1, lane + 2, lane + 3}, b = {lane * 3, 7, 9, lane};
  const i32x8 a8 = {lane, 1, 2, 3, 4, 5, 6, 7}, b8 = {7, 6, 5, 4, 3, 2, 1, lane};
  i32x16 c0 = {0}, c1 = {0};
  f32x16 f0 = {0}, f1 = {0};
  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = lane + j;
  const float k0 = 0.999f, k1 = 0.001f;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  if (role != 0) {
    for (int i = 0; i < kCoIter; ++i) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (role & 1) {
          if constexpr (QK == 0) {
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
          } else {
            f0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, f0, 0, 0, 0, 0, 0, 0);
            f1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b8, a8, f1, 0, 0, 0, 0, 0, 0);
          }
        }
        if (role & 2) {
#pragma unroll
          for (int v = 0; v < VPM; v += 16) valu16(x, k0, k1);
        }
      }
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  int acc = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc += c0[e] + c1[e] + (int)f0[e] + (int)f1[e];
  float xs = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) xs += x[j];
  out[blockIdx.x * 512 + threadIdx.x] = (uint32_t)acc + __float_as_uint(xs);
  if (lane == 0) cyc[blockIdx.x * 8 + wave] = t1 - t0;
}

typedef void (*CoFn)(uint32_t*, uint64_t*, int);
struct CoVariant {
  const char* name;
  CoFn fn;
};
const CoVariant kCoVariants[] = {
    {"i8 32x32x32 chains, 16 FMA per MFMA pair", coexec_kernel<0, 16>},
    {"i8 32x32x32 chains, 32 FMA per MFMA pair", coexec_kernel<0, 32>},
    {"f8f6f4 32x32x64 chains, 16 FMA per MFMA pair", coexec_kernel<1, 16>},
    {"f8f6f4 32x32x64 chains, 32 FMA per MFMA pair", coexec_kernel<1, 32>},
};
constexpr int kNumCoVariants = sizeof(kCoVariants) / sizeof(kCoVariants[0]);
struct CoMode {
  const char* name;
  int mode;
};
const CoMode kCoModes[] = {
    {"MFMA stream alone", 1},
    {"VALU stream alone", 2 << 2},
    {"MFMA wave beside VALU wave", 1 | (2 << 2)},
    {"both streams in one wave", 3},
    {"both streams in each of two waves", 3 | (3 << 2)},
};
constexpr int kNumCoModes = sizeof(kCoModes) / sizeof(kCoModes[0]);
constexpr int kCus = 256;

thread_local char g_err[256];

int fail(const char* what, hipError_t e) {
  snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
  return -1;
}

}  // namespace

extern "C" {

const char* sage_probe_last_error() { return g_err; }
int sage_probe_issue_count() { return kNumIssue; }
const char* sage_probe_issue_name(int i) { return i >= 0 && i < kNumIssue ? kIssue[i].name : ""; }
int sage_probe_coexec_count() { return kNumCoVariants * kNumCoModes; }
const char* sage_probe_coexec_variant(int i) {
  return i >= 0 && i < kNumCoVariants * kNumCoModes ? kCoVariants[i / kNumCoModes].name : "";
}
const char* sage_probe_coexec_mode(int i) {
  return i >= 0 && i < kNumCoVariants * kNumCoModes ? kCoModes[i % kNumCoModes].name : "";
}

// ticks[2 * i + w - 1]: ticks per wave-instruction of probe i with about w
// waves per SIMD (w = 1, 2).  Returns the number of probes, or -1.
int sage_probe_issue(double* ticks, int cap) {
  if (ticks == nullptr || cap < 2 * kNumIssue) {
    snprintf(g_err, sizeof(g_err), "ticks must hold %d values", 2 * kNumIssue);
    return -1;
  }
  const int max_blocks = 2 * kCus;
  uint32_t* out = nullptr;
  uint64_t* cyc = nullptr;
  hipError_t e = hipMalloc(&out, (size_t)max_blocks * 256 * 4);
  if (e != hipSuccess) return fail("hipMalloc", e);
  e = hipMalloc(&cyc, (size_t)max_blocks * 4 * 8);
  if (e != hipSuccess) {
    (void)hipFree(out);
    return fail("hipMalloc", e);
  }
  uint64_t* hc = new uint64_t[(size_t)max_blocks * 4];
  int rc = kNumIssue;
  for (int w = 1; w <= 2 && rc > 0; ++w) {
    const int blocks = w * kCus;
    for (int i = 0; i < kNumIssue; ++i) {
      hipLaunchKernelGGL(kIssue[i].fn, dim3(blocks), dim3(256), 0, 0, out, cyc, 1.0001f);  // warm
      hipLaunchKernelGGL(kIssue[i].fn, dim3(blocks), dim3(256), 0, 0, out, cyc, 1.0001f);
      e = hipDeviceSynchronize();
      if (e == hipSuccess) e = hipMemcpy(hc, cyc, (size_t)blocks * 4 * 8, hipMemcpyDeviceToHost);
      if (e != hipSuccess) {
        rc = fail("issue probe", e);
        break;
      }
      double s = 0.0;
      for (int j = 0; j < blocks * 4; ++j) s += (double)hc[j];
      ticks[2 * i + w - 1] = s / (blocks * 4.0) / (kIssueIter * 8.0);
    }
  }
  delete[] hc;
  (void)hipFree(out);
  (void)hipFree(cyc);
  return rc;
}

// ticks[2 * i], ticks[2 * i + 1]: mean ticks per iteration (four MFMA pairs
// and their FMAs) of waves 0-3 and 4-7 for row i (variant i / modes, mode
// i % modes).  Returns the number of rows, or -1.
int sage_probe_coexec(double* ticks, int cap) {
  const int rows = kNumCoVariants * kNumCoModes;
  if (ticks == nullptr || cap < 2 * rows) {
    snprintf(g_err, sizeof(g_err), "ticks must hold %d values", 2 * rows);
    return -1;
  }
  uint32_t* out = nullptr;
  uint64_t* cyc = nullptr;
  hipError_t e = hipMalloc(&out, (size_t)kCus * 512 * 4);
  if (e != hipSuccess) return fail("hipMalloc", e);
  e = hipMalloc(&cyc, (size_t)kCus * 8 * 8);
  if (e != hipSuccess) {
    (void)hipFree(out);
    return fail("hipMalloc", e);
  }
  uint64_t* hc = new uint64_t[(size_t)kCus * 8];
  int rc = rows;
  for (int i = 0; i < rows; ++i) {
    const CoFn fn = kCoVariants[i / kNumCoModes].fn;
    const int mode = kCoModes[i % kNumCoModes].mode;
    hipLaunchKernelGGL(fn, dim3(kCus), dim3(512), 0, 0, out, cyc, mode);  // warm
    hipLaunchKernelGGL(fn, dim3(kCus), dim3(512), 0, 0, out, cyc, mode);
    e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(hc, cyc, (size_t)kCus * 8 * 8, hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
      rc = fail("co-execution probe", e);
      break;
    }
    double lo = 0.0, hi = 0.0;
    for (int b = 0; b < kCus; ++b)
      for (int w = 0; w < 8; ++w) (w < 4 ? lo : hi) += (double)hc[b * 8 + w];
    ticks[2 * i] = lo / (kCus * 4.0 * kCoIter);
    ticks[2 * i + 1] = hi / (kCus * 4.0 * kCoIter);
  }
  delete[] hc;
  (void)hipFree(out);
  (void)hipFree(cyc);
  return rc;
}

}  // extern "C"
