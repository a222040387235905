// extern "C" boundary of libsage_mi355x.so: argument validation, error
// reporting and dispatch to the gfx950 kernels.  See include/sage_mi355x.h.
#include <stdio.h>
#include <stdarg.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdlib>
#include <mutex>

#include "../../include/sage_mi355x.h"
#include "sage_common.h"

#include "sage_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kAttnMaxN = (int64_t)1 << 22;  // sage_attn_fwd's sequence-length limit
// Workgroups of one 1D launch of 256-thread workgroups (the dispatch packet
// holds the grid in work-items, a 32-bit count).
constexpr int64_t kMaxGridUnits = ((int64_t)1 << 24) - 1;

int check_common(int64_t bh, int64_t n, int64_t d, int qk, int pv, int gran) {
  if (bh <= 0 || n <= 0) return fail(SAGE_ERR_ARG, "bh=%lld and n=%lld must be positive", (long long)bh, (long long)n);
  if (d != 64 && d != 128) return fail(SAGE_ERR_ARG, "head_dim must be 64 or 128, got %lld", (long long)d);
  if (qk != SAGE_QK_INT8 && qk != SAGE_QK_FP8) return fail(SAGE_ERR_ARG, "unknown qk_kind %d", qk);
  if (pv != SAGE_PV_BF16 && pv != SAGE_PV_FP8) return fail(SAGE_ERR_ARG, "unknown pv_kind %d", pv);
  if (gran != SAGE_GRAN_TOKEN && gran != SAGE_GRAN_BLOCK64) return fail(SAGE_ERR_ARG, "unknown granularity %d", gran);
  if (bh > 65535) return fail(SAGE_ERR_ARG, "bh=%lld exceeds the grid limit 65535", (long long)bh);
  if (n > (int64_t)1 << 24) return fail(SAGE_ERR_ARG, "n=%lld exceeds 2^24", (long long)n);
  return SAGE_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SAGE_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  g_err[0] = '\0';
  return SAGE_OK;
}

}  // namespace

extern "C" {

int sage_abi_version(void) { return SAGE_ABI_VERSION; }

const char* sage_last_error(void) { return g_err; }

int64_t sage_padded_len(int64_t n) { return sage::padded_len(n); }

size_t sage_quant_workspace_bytes(int64_t bh, int64_t n, int64_t d) { return sage::quant_workspace_bytes(bh, n, d); }

size_t sage_attn_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d) {
  return sage::attn_workspace_bytes(b, h, n, d);
}

size_t sage_attn_masked_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d) {
  return sage::attn_workspace_bytes(b, h, n, d, true);
}

}  // extern "C"

namespace {

// Outputs and workspace of a quantization call.
int check_quant_outputs(int64_t bh, int64_t n, int64_t d, int64_t h_producer, int pv_kind, int smooth_k,
                        const void* q_codes,
                        const float* q_scale, const void* k_codes, const float* k_scale, const void* v_out,
                        const float* v_scale, const void* k_mean, const void* workspace, size_t workspace_bytes) {
  if (!q_codes || !q_scale || !k_codes || !k_scale || !v_out) return fail(SAGE_ERR_ARG, "null tensor pointer");
  if (pv_kind == SAGE_PV_FP8 && !v_scale) return fail(SAGE_ERR_ARG, "fp8 PV needs v_scale");
  const void* ptrs[] = {q_codes, q_scale, k_codes, k_scale, v_out};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(SAGE_ERR_ALIGN, "tensor pointers must be 16-byte aligned");
  if (v_scale && !aligned16(v_scale)) return fail(SAGE_ERR_ALIGN, "v_scale must be 16-byte aligned");
  const int64_t units = sage::quant_grid_units(bh, n, d, h_producer);
  if (units > kMaxGridUnits)
    return fail(SAGE_ERR_ARG, "quantizing bh=%lld x n=%lld takes %lld workgroups, beyond one launch's %lld",
                (long long)bh, (long long)n, (long long)units, (long long)kMaxGridUnits);
  if (smooth_k) {
    if (!k_mean) return fail(SAGE_ERR_ARG, "smooth_k needs k_mean");
    const size_t need = sage::quant_workspace_bytes(bh, n, d);
    if (!workspace || workspace_bytes < need)
      return fail(SAGE_ERR_WORKSPACE, "workspace of %zu bytes needed, got %zu", need, workspace_bytes);
    if (!aligned16(workspace)) return fail(SAGE_ERR_ALIGN, "workspace must be 16-byte aligned");
  }
  return SAGE_OK;
}

// Inputs of the q/k/v producer.
int check_producer(const void* qkv, const float* q_norm_w, const float* k_norm_w, const float* freqs, int64_t b,
                   int64_t h, int64_t n, int64_t d, float norm_eps, sage::ProdArgs& prod) {
  if (b <= 0 || h <= 0) return fail(SAGE_ERR_ARG, "b=%lld and h=%lld must be positive", (long long)b, (long long)h);
  if (b * h > 65535) return fail(SAGE_ERR_ARG, "b*h=%lld exceeds the grid limit 65535", (long long)(b * h));
  if (n <= 0) return fail(SAGE_ERR_ARG, "n=%lld must be positive", (long long)n);
  if (n > (int64_t)1 << 24) return fail(SAGE_ERR_ARG, "n=%lld exceeds 2^24", (long long)n);
  if (d != 64 && d != 128) return fail(SAGE_ERR_ARG, "head_dim must be 64 or 128, got %lld", (long long)d);
  if (!qkv || !q_norm_w || !k_norm_w || !freqs) return fail(SAGE_ERR_ARG, "null tensor pointer");
  const void* ptrs[] = {qkv, q_norm_w, k_norm_w, freqs};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(SAGE_ERR_ALIGN, "tensor pointers must be 16-byte aligned");
  if (!(norm_eps >= 0.0f)) return fail(SAGE_ERR_ARG, "norm_eps must be >= 0");
  // the producer's backward: one workgroup per (64-token block, head) in a 1D grid
  if (b * h * ((n + 63) / 64) > kMaxGridUnits)
    return fail(SAGE_ERR_ARG, "b*h*ceil(n/64) = %lld exceeds the grid limit", (long long)(b * h * ((n + 63) / 64)));
  // the standalone producer: one per (pass of 256/(d/8) tokens, group of kSlabHeads heads)
  const int64_t rpp = 256 / (d / 8);
  const int64_t slabs = b * ((n + rpp - 1) / rpp) * ((h + sage::kSlabHeads - 1) / sage::kSlabHeads);
  if (slabs > kMaxGridUnits)
    return fail(SAGE_ERR_ARG, "%lld producer slabs exceed the grid limit", (long long)slabs);
  // 256 token rows of the projection output (3*h*d bf16 each) within 32-bit byte offsets
  if (3 * h * d * 2 * 256 > (int64_t)0xffffffff)
    return fail(SAGE_ERR_ARG, "3*h*d = %lld channels per token row is too wide for the producer", (long long)(3 * h * d));
  prod = sage::ProdArgs{static_cast<const uint16_t*>(qkv), q_norm_w, k_norm_w, freqs, (int)h, (int)(b * h),
                        norm_eps};
  return SAGE_OK;
}

// Backward workspace: byte offsets of the quantization's outputs (codes,
// scales, K mean, column-sum partials), the T images of dO, Q and K~, and D.
struct BwdWorkspace {
  size_t qc, qs, kc, ks, kmean, quant, tdo, tq, tk, rdo, rv, delta, sums, dq_part, dq_ctr, bytes;
};

BwdWorkspace bwd_workspace(int64_t b, int64_t bh, int64_t n, int64_t d) {
  const size_t np = (size_t)sage::padded_len(n), rows = (size_t)bh * np;
  BwdWorkspace w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = (off + bytes + 255) & ~(size_t)255;
    return at;
  };
  w.qc = take(rows * d);
  w.qs = take(rows * 4);
  w.kc = take(rows * d);
  w.ks = take(rows * 4);
  w.kmean = take((size_t)bh * d * 2);
  w.quant = take(sage::quant_workspace_bytes(bh, n, d));
  w.tdo = take(rows * d * 2);
  w.tq = take(rows * d * 2);
  w.tk = take(rows * d * 2);
  w.rdo = take(rows * d * 2);
  w.rv = take(rows * d * 2);
  w.delta = take(rows * 4);
  // document-id summaries (used with doc_ids): key tiles, 32- and 128-row blocks
  w.sums = take((size_t)b * ((n + 63) / 64 + np / 32 + np / 128) * sizeof(int4));
  // fp32 partial dQ of the cut items' two key-tile halves, their counters
  w.dq_part = take((size_t)sage::kBwdDqSplit * 2 * 128 * d * sizeof(float));
  w.dq_ctr = take((size_t)sage::kBwdDqSplit * sizeof(uint64_t));
  w.bytes = off;
  return w;
}

}  // namespace

extern "C" {

int sage_quantize_qkv(const void* q, const void* k, const void* v, int64_t bh, int64_t n, int64_t d, int qk_kind,
                      int pv_kind, int granularity, int smooth_k, float sm_scale_log2e, void* q_codes,
                      float* q_scale, void* k_codes, float* k_scale, void* v_out, float* v_scale, void* k_mean,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = check_common(bh, n, d, qk_kind, pv_kind, granularity);
  if (st) return st;
  if (!q || !k || !v) return fail(SAGE_ERR_ARG, "null tensor pointer");
  const void* ins[] = {q, k, v};
  for (const void* p : ins)
    if (!aligned16(p)) return fail(SAGE_ERR_ALIGN, "tensor pointers must be 16-byte aligned");
  st = check_quant_outputs(bh, n, d, 0, pv_kind, smooth_k, q_codes, q_scale, k_codes, k_scale, v_out, v_scale, k_mean,
                           workspace, workspace_bytes);
  if (st) return st;
  hipError_t e = sage::launch_quantize(
      qk_kind, pv_kind, granularity, smooth_k != 0, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
      static_cast<const uint16_t*>(v), bh, n, d, sm_scale_log2e, static_cast<double*>(workspace),
      static_cast<uint8_t*>(q_codes), q_scale, static_cast<uint8_t*>(k_codes), k_scale, static_cast<uint8_t*>(v_out),
      v_scale, static_cast<uint16_t*>(k_mean), sage::ProdArgs{}, stream);
  return launch_status(e, "sage_quantize_qkv");
}

int sage_qkv_postprocess(const void* qkv, const float* q_norm_w, const float* k_norm_w, const float* freqs,
                         int64_t b, int64_t h, int64_t n, int64_t d, float norm_eps, void* q_out, void* k_out,
                         void* v_out, hipStream_t stream) {
  sage::ProdArgs prod;
  int st = check_producer(qkv, q_norm_w, k_norm_w, freqs, b, h, n, d, norm_eps, prod);
  if (st) return st;
  if (!q_out || !k_out || !v_out) return fail(SAGE_ERR_ARG, "null tensor pointer");
  const void* outs[] = {q_out, k_out, v_out};
  for (const void* p : outs)
    if (!aligned16(p)) return fail(SAGE_ERR_ALIGN, "tensor pointers must be 16-byte aligned");
  return launch_status(sage::launch_qkv_postprocess(prod, b * h, n, d, static_cast<uint16_t*>(q_out),
                                                    static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out),
                                                    stream),
                       "sage_qkv_postprocess");
}

int sage_qkv_postprocess_bwd(const void* qkv, const float* q_norm_w, const float* k_norm_w, const float* freqs,
                             const void* grad_q, const void* grad_k, const void* grad_v, int64_t b, int64_t h,
                             int64_t n, int64_t d, float norm_eps, void* dqkv, hipStream_t stream) {
  sage::ProdArgs prod;
  int st = check_producer(qkv, q_norm_w, k_norm_w, freqs, b, h, n, d, norm_eps, prod);
  if (st) return st;
  if (!grad_q || !grad_k || !grad_v || !dqkv) return fail(SAGE_ERR_ARG, "null tensor pointer");
  const void* ptrs[] = {grad_q, grad_k, grad_v, dqkv};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(SAGE_ERR_ALIGN, "tensor pointers must be 16-byte aligned");
  return launch_status(sage::launch_qkv_postprocess_bwd(prod, b * h, n, d, static_cast<const uint16_t*>(grad_q),
                                                        static_cast<const uint16_t*>(grad_k),
                                                        static_cast<const uint16_t*>(grad_v),
                                                        static_cast<uint16_t*>(dqkv), stream),
                       "sage_qkv_postprocess_bwd");
}

int sage_quantize_from_qkv(const void* qkv, const float* q_norm_w, const float* k_norm_w, const float* freqs,
                           int64_t b, int64_t h, int64_t n, int64_t d, float norm_eps, int qk_kind, int pv_kind,
                           int granularity, int smooth_k, float sm_scale_log2e, void* q_codes, float* q_scale,
                           void* k_codes, float* k_scale, void* v_out, float* v_scale, void* k_mean, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  sage::ProdArgs prod;
  int st = check_producer(qkv, q_norm_w, k_norm_w, freqs, b, h, n, d, norm_eps, prod);
  if (st) return st;
  st = check_common(b * h, n, d, qk_kind, pv_kind, granularity);
  if (st) return st;
  st = check_quant_outputs(b * h, n, d, h, pv_kind, smooth_k, q_codes, q_scale, k_codes, k_scale, v_out, v_scale,
                           k_mean, workspace, workspace_bytes);
  if (st) return st;
  hipError_t e = sage::launch_quantize(
      qk_kind, pv_kind, granularity, smooth_k != 0, nullptr, nullptr, nullptr, b * h, n, d, sm_scale_log2e,
      static_cast<double*>(workspace), static_cast<uint8_t*>(q_codes), q_scale, static_cast<uint8_t*>(k_codes),
      k_scale, static_cast<uint8_t*>(v_out), v_scale, static_cast<uint16_t*>(k_mean), prod, stream);
  return launch_status(e, "sage_quantize_from_qkv");
}

}  // extern "C"

namespace {

// A 56-bit tag never passed to an earlier attention launch of this process (a
// clock reading at first use, plus a call counter): the split items' arrival
// counters of other calls never match it (AttnParams::merge_ctr).
uint64_t next_merge_tag() {
  static std::atomic<uint64_t> counter{0};
  static const uint64_t base =
      (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count() * 0x9E3779B97F4A7C15ull;
  return (base + counter.fetch_add(1, std::memory_order_relaxed) * 2 + 1) & (((uint64_t)1 << 56) - 1);
}

// The split items of unmasked launches merge in the attention kernel, unless
// SAGE_MERGE=kernel asks for the separate merge kernel (tests compare both).
bool merge_in_kernel() {
  const char* e = std::getenv("SAGE_MERGE");
  return e == nullptr || strcmp(e, "kernel") != 0;
}

// The backward cuts its last dQ items in two key halves unless
// SAGE_BWD_SPLIT=off (tests compare both).
bool bwd_split_enabled() {
  const char* e = std::getenv("SAGE_BWD_SPLIT");
  return e == nullptr || strcmp(e, "off") != 0;
}

// sage_attn_fwd and its variants: validation, workspace layout and launch.
// s_dump (int8 QK, per-token scales, no mask only) receives the S^T
// accumulators the kernel's loop consumes.
int attn_fwd_impl(const void* q_codes, const float* q_scale, const void* k_codes, const float* k_scale,
                  const void* v_in, const float* v_scale, int64_t b, int64_t h, int64_t n, int64_t d, int qk_kind,
                  int pv_kind, int granularity, const uint8_t* tile_mask, int64_t mask_stride_z, int64_t mask_nq,
                  int64_t mask_nkv, const int32_t* doc_ids, void* workspace, size_t workspace_bytes, void* out,
                  int out_layout, float* lse, int32_t* s_dump, const char* name, hipStream_t stream) {
  if (b <= 0 || h <= 0) return fail(SAGE_ERR_ARG, "b=%lld and h=%lld must be positive", (long long)b, (long long)h);
  int st = check_common(b * h, n, d, qk_kind, pv_kind, granularity);
  if (st) return st;
  if (!q_codes || !q_scale || !k_codes || !k_scale || !v_in || !out || !lse)
    return fail(SAGE_ERR_ARG, "null tensor pointer");
  if (pv_kind == SAGE_PV_FP8 && !v_scale) return fail(SAGE_ERR_ARG, "fp8 PV needs v_scale");
  const void* ptrs[] = {q_codes, q_scale, k_codes, k_scale, v_in, out};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(SAGE_ERR_ALIGN, "tensor pointers must be 16-byte aligned");
  if (v_scale && !aligned16(v_scale)) return fail(SAGE_ERR_ALIGN, "v_scale must be 16-byte aligned");
  if (out_layout != SAGE_OUT_BHND && out_layout != SAGE_OUT_BNHD)
    return fail(SAGE_ERR_ARG, "out_layout must be 0 ([B,H,N,D]) or 1 ([B,N,H,D]), got %d", out_layout);
  // one head's operands are addressed through buffer resources with 32-bit
  // byte offsets: Np*D*2 bytes of bf16 V must stay below 2^31
  if (n > kAttnMaxN) return fail(SAGE_ERR_ARG, "n=%lld exceeds %lld for the attention", (long long)n, (long long)kAttnMaxN);
  // The epilogue addresses 32 output rows of one head in 32-bit byte offsets:
  // at most 32 * h*d*2 bytes, under 2^31 since b*h <= 65535 and d <= 128.
  const int64_t nq = (n + 127) / 128, nkv = (n + 63) / 64;
  int mask = 0;
  if (tile_mask) {
    if (mask_nq != nq || mask_nkv != nkv)
      return fail(SAGE_ERR_ARG, "block_mask must be %lld x %lld tiles, got %lld x %lld", (long long)nq,
                  (long long)nkv, (long long)mask_nq, (long long)mask_nkv);
    if (mask_stride_z != 0 && mask_stride_z != nq * nkv)
      return fail(SAGE_ERR_ARG, "mask_stride_z must be 0 (2D mask) or %lld (3D mask)", (long long)(nq * nkv));
    mask |= 1;
  }
  if (doc_ids) mask |= 2;
  sage::AttnParams p;
  memset(&p, 0, sizeof(p));
  // masked launches cut no item, so they need no partial slots
  const sage::AttnWorkspace ws = sage::attn_workspace(b, h, n, d, mask != 0);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(SAGE_ERR_WORKSPACE, "workspace of %zu bytes needed, got %zu", ws.bytes, workspace_bytes);
  if (!aligned16(workspace)) return fail(SAGE_ERR_ALIGN, "workspace must be 16-byte aligned");
  uint8_t* wsp = static_cast<uint8_t*>(workspace);
  if (doc_ids) {
    const int64_t nt = nkv;
    p.kv_sum = reinterpret_cast<const int4*>(wsp + ws.doc_off);
    p.q_sum = p.kv_sum + b * nt;
    p.q_sum128 = p.q_sum + b * (sage::padded_len(n) / 32);
    p.doc_range = p.q_sum128 + b * (sage::padded_len(n) / 128);
    p.heavy = reinterpret_cast<int4*>(wsp + ws.heavy_off);
    p.heavy_max = sage::kHeavyMax;
  }
  p.qc = static_cast<const uint8_t*>(q_codes);
  p.qs = q_scale;
  p.kc = static_cast<const uint8_t*>(k_codes);
  p.ks = k_scale;
  p.vin = static_cast<const uint8_t*>(v_in);
  p.vs = v_scale;
  p.tile_mask = tile_mask;
  p.mask_stride_z = mask_stride_z;
  p.mask_nkv = mask_nkv;
  p.doc = doc_ids;
  p.out = static_cast<uint16_t*>(out);
  if (out_layout == SAGE_OUT_BNHD) {
    p.out_bs = n * h * d;
    p.out_hs = d;
    p.out_rs = h * d;
  } else {
    p.out_bs = h * n * d;
    p.out_hs = n * d;
    p.out_rs = d;
  }
  p.lse = lse;
  p.n = n;
  p.np = sage::padded_len(n);
  p.h = (int)h;
  p.bh = (int)(b * h);
  p.nt = (int)nkv;
  p.light_last = (nq > 1 && n - (nq - 1) * 128 <= 64) ? 1 : 0;
  // unmasked launches cut the items of the last, partial dispatch round
  p.n_whole = (int)(b * h * nq);
  p.split_parts = 1;
  if (mask == 0) {
    p.n_whole = (int)ws.split.whole;
    p.split_parts = ws.split.parts;
    p.part = reinterpret_cast<float*>(wsp + ws.part_off);
    if (ws.split.parts > 1 && merge_in_kernel()) {
      p.merge_ctr = reinterpret_cast<uint64_t*>(wsp + ws.ctr_off);
      p.merge_tag = next_merge_tag();
    }
  }
  if ((int64_t)p.bh * nq + (int64_t)sage::kHeavyMax * h + 8 * sage::kResidentWGs > kMaxGridUnits)
    return fail(SAGE_ERR_ARG, "b*h*ceil(n/128) = %lld exceeds the grid limit", (long long)(p.bh * nq));
  p.s_dump = s_dump;
  hipError_t e = sage::launch_attn(qk_kind, pv_kind, granularity, mask, p, d, (int)b, stream);
  return launch_status(e, name);
}

}  // namespace

extern "C" {

int sage_attn_fwd(const void* q_codes, const float* q_scale, const void* k_codes, const float* k_scale,
                  const void* v_in, const float* v_scale, int64_t b, int64_t h, int64_t n, int64_t d, int qk_kind,
                  int pv_kind, int granularity, const uint8_t* tile_mask, int64_t mask_stride_z, int64_t mask_nq,
                  int64_t mask_nkv, const int32_t* doc_ids, void* workspace, size_t workspace_bytes, void* out,
                  int out_layout, float* lse, hipStream_t stream) {
  return attn_fwd_impl(q_codes, q_scale, k_codes, k_scale, v_in, v_scale, b, h, n, d, qk_kind, pv_kind, granularity,
                       tile_mask, mask_stride_z, mask_nq, mask_nkv, doc_ids, workspace, workspace_bytes, out,
                       out_layout, lse, nullptr, "sage_attn_fwd", stream);
}

}  // extern "C"

namespace {

// Device scratch of sage_attn_fwd_noalloc: the document-id summaries and the
// split-tail partials that sage_attn_fwd keeps in its workspace argument.
// Each GPU the library runs on holds its own copy until the process ends.
// Host code never uses the array's name as an address: its device address
// comes from hipGetSymbolAddress, once per device, with that device current.
__device__ __align__(256) uint8_t scratch[SAGE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Scratch address on the device of `stream`, which must be the current device.
int scratch_of_stream(hipStream_t stream, void** ptr) {
  int cur = -1, sdev = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess) e = hipStreamGetDevice(stream, &sdev);
  if (e != hipSuccess) return fail(SAGE_ERR_LAUNCH, "device of the stream: %s", hipGetErrorString(e));
  if (sdev != cur)
    return fail(SAGE_ERR_ARG, "the stream belongs to device %d, the current device is %d", sdev, cur);
  if (cur < 0 || cur >= kMaxDevices) return fail(SAGE_ERR_ARG, "device %d beyond the first %d", cur, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[cur]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(SAGE_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_ptr[cur] = p;
  }
  *ptr = g_scratch_ptr[cur];
  return SAGE_OK;
}

}  // namespace

extern "C" {

int sage_attn_fwd_noalloc(const void* q_codes, const float* q_scale, const void* k_codes, const float* k_scale,
                          const void* v_in, const float* v_scale, int64_t b, int64_t h, int64_t n, int64_t d,
                          int qk_kind, int pv_kind, int granularity, const uint8_t* tile_mask, int64_t mask_stride_z,
                          int64_t mask_nq, int64_t mask_nkv, const int32_t* doc_ids, void* out, int out_layout,
                          float* lse, hipStream_t stream) {
  if (b <= 0 || h <= 0) return fail(SAGE_ERR_ARG, "b=%lld and h=%lld must be positive", (long long)b, (long long)h);
  int st = check_common(b * h, n, d, qk_kind, pv_kind, granularity);
  if (st) return st;
  const size_t need = sage::attn_workspace_bytes(b, h, n, d, tile_mask != nullptr || doc_ids != nullptr);
  if (need > (size_t)SAGE_NOALLOC_SCRATCH_BYTES)
    return fail(SAGE_ERR_WORKSPACE,
                "b=%lld h=%lld n=%lld d=%lld needs %zu bytes of workspace, beyond the %zu-byte scratch of the "
                "allocation-free entry point; use sage_attn_fwd with a workspace",
                (long long)b, (long long)h, (long long)n, (long long)d, need, (size_t)SAGE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  st = scratch_of_stream(stream, &ws);
  if (st) return st;
  return attn_fwd_impl(q_codes, q_scale, k_codes, k_scale, v_in, v_scale, b, h, n, d, qk_kind, pv_kind, granularity,
                       tile_mask, mask_stride_z, mask_nq, mask_nkv, doc_ids, ws, SAGE_NOALLOC_SCRATCH_BYTES, out,
                       out_layout, lse, nullptr, "sage_attn_fwd_noalloc", stream);
}

int sage_attn_qk_accumulators(const void* q_codes, const float* q_scale, const void* k_codes, const float* k_scale,
                              const void* v_in, const float* v_scale, int64_t b, int64_t h, int64_t n, int64_t d,
                              int qk_kind, int pv_kind, void* workspace, size_t workspace_bytes, void* out, float* lse,
                              int32_t* s_out, hipStream_t stream) {
  if (!s_out) return fail(SAGE_ERR_ARG, "null tensor pointer");
  return attn_fwd_impl(q_codes, q_scale, k_codes, k_scale, v_in, v_scale, b, h, n, d, qk_kind, pv_kind,
                       SAGE_GRAN_TOKEN, nullptr, 0, 0, 0, nullptr, workspace, workspace_bytes, out, SAGE_OUT_BHND,
                       lse, s_out, "sage_attn_qk_accumulators", stream);
}

size_t sage_attn_bwd_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d) {
  return bwd_workspace(b, b * h, n, d).bytes;
}

int sage_attn_bwd(const void* q, const void* k, const void* v, const void* out, const float* lse, const void* dout,
                  int64_t b, int64_t h, int64_t n, int64_t d, int qk_kind, int smooth_k, float sm_scale,
                  float sm_scale_log2e, const uint8_t* tile_mask, int64_t mask_stride_z, int64_t mask_nq, int64_t mask_nkv,
                  const int32_t* doc_ids, void* workspace, size_t workspace_bytes, void* dq, void* dk, void* dv,
                  hipStream_t stream) {
  if (b <= 0 || h <= 0) return fail(SAGE_ERR_ARG, "b=%lld and h=%lld must be positive", (long long)b, (long long)h);
  int st = check_common(b * h, n, d, qk_kind, SAGE_PV_BF16, SAGE_GRAN_TOKEN);
  if (st) return st;
  if (!q || !k || !v || !out || !lse || !dout || !dq || !dk || !dv) return fail(SAGE_ERR_ARG, "null tensor pointer");
  const void* ptrs[] = {q, k, v, out, dout, dq, dk, dv};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(SAGE_ERR_ALIGN, "tensor pointers must be 16-byte aligned");
  if (!(sm_scale > 0.0f) || !(sm_scale_log2e > 0.0f))
    return fail(SAGE_ERR_ARG, "sm_scale and sm_scale_log2e must be positive");
  const int64_t nq = (n + 127) / 128, nkv = (n + 63) / 64;
  int mask = 0;
  if (tile_mask) {
    if (mask_nq != nq || mask_nkv != nkv)
      return fail(SAGE_ERR_ARG, "block_mask must be %lld x %lld tiles, got %lld x %lld", (long long)nq,
                  (long long)nkv, (long long)mask_nq, (long long)mask_nkv);
    if (mask_stride_z != 0 && mask_stride_z != nq * nkv)
      return fail(SAGE_ERR_ARG, "mask_stride_z must be 0 (2D mask) or %lld (3D mask)", (long long)(nq * nkv));
    mask |= 1;
  }
  if (doc_ids) mask |= 2;
  // the dK/dV and dQ launches: 512-thread workgroups, one per 128-row tile
  if ((b * h) * ((n + 127) / 128) > kMaxGridUnits / 2)
    return fail(SAGE_ERR_ARG, "b*h*ceil(n/128) = %lld exceeds the grid limit", (long long)(b * h * ((n + 127) / 128)));
  if (sage::quant_grid_units(b * h, n, d, 0) > kMaxGridUnits)
    return fail(SAGE_ERR_ARG, "quantizing b*h=%lld x n=%lld exceeds one launch's %lld workgroups", (long long)(b * h),
                (long long)n, (long long)kMaxGridUnits);
  const BwdWorkspace ws = bwd_workspace(b, b * h, n, d);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(SAGE_ERR_WORKSPACE, "workspace of %zu bytes needed, got %zu", ws.bytes, workspace_bytes);
  if (!aligned16(workspace)) return fail(SAGE_ERR_ALIGN, "workspace must be 16-byte aligned");
  uint8_t* w = static_cast<uint8_t*>(workspace);
  const int64_t bh = b * h;
  const auto* q16 = static_cast<const uint16_t*>(q);
  const auto* k16 = static_cast<const uint16_t*>(k);
  const auto* do16 = static_cast<const uint16_t*>(dout);
  // codes, scales and the K mean of the forward's per-token quantization;
  // dO takes the place of V, so the bf16 "V operand" written is dO's T image
  hipError_t e = sage::launch_quantize(
      qk_kind, SAGE_PV_BF16, SAGE_GRAN_TOKEN, smooth_k != 0, q16, k16, do16, bh, n, d,
      sm_scale_log2e, reinterpret_cast<double*>(w + ws.quant), w + ws.qc,
      reinterpret_cast<float*>(w + ws.qs), w + ws.kc, reinterpret_cast<float*>(w + ws.ks), w + ws.tdo, nullptr,
      reinterpret_cast<uint16_t*>(w + ws.kmean), sage::ProdArgs{}, stream);
  if (e != hipSuccess) return launch_status(e, "sage_attn_bwd (quantize)");
  sage::TImageJobs jobs{};
  jobs.x[0] = q16;
  jobs.out[0] = reinterpret_cast<uint16_t*>(w + ws.tq);
  jobs.x[1] = k16;
  jobs.mu[1] = smooth_k ? reinterpret_cast<const uint16_t*>(w + ws.kmean) : nullptr;
  jobs.out[1] = reinterpret_cast<uint16_t*>(w + ws.tk);
  sage::TImageJobs rjobs{};
  rjobs.x[0] = do16;
  rjobs.out[0] = reinterpret_cast<uint16_t*>(w + ws.rdo);
  rjobs.x[1] = static_cast<const uint16_t*>(v);
  rjobs.out[1] = reinterpret_cast<uint16_t*>(w + ws.rv);
  e = sage::launch_bwd_prep(jobs, rjobs, do16, static_cast<const uint16_t*>(out), bh, n, d,
                            reinterpret_cast<float*>(w + ws.delta), stream);
  if (e != hipSuccess) return launch_status(e, "sage_attn_bwd (prep)");
  const int4* sums = reinterpret_cast<const int4*>(w + ws.sums);
  const int64_t np = sage::padded_len(n);
  if (doc_ids) {
    e = sage::launch_doc_summaries(doc_ids, n, (int)b, const_cast<int4*>(sums), const_cast<int4*>(sums + b * nkv),
                                   const_cast<int4*>(sums + b * nkv + b * (np / 32)), nullptr, stream);
    if (e != hipSuccess) return launch_status(e, "sage_attn_bwd (summaries)");
  }
  sage::BwdParams p;
  memset(&p, 0, sizeof(p));
  p.qc = w + ws.qc;
  p.qs = reinterpret_cast<const float*>(w + ws.qs);
  p.kc = w + ws.kc;
  p.ks = reinterpret_cast<const float*>(w + ws.ks);
  p.v = static_cast<const uint16_t*>(v);
  p.dout = do16;
  p.tq = reinterpret_cast<const uint16_t*>(w + ws.tq);
  p.tk = reinterpret_cast<const uint16_t*>(w + ws.tk);
  p.tdo = reinterpret_cast<const uint16_t*>(w + ws.tdo);
  p.rdo = reinterpret_cast<const uint16_t*>(w + ws.rdo);
  p.rv = reinterpret_cast<const uint16_t*>(w + ws.rv);
  p.lse = lse;
  p.delta = reinterpret_cast<const float*>(w + ws.delta);
  p.tile_mask = tile_mask;
  p.mask_stride_z = mask_stride_z;
  p.mask_nkv = mask_nkv;
  p.doc = doc_ids;
  p.kv_sum = sums;
  p.q_sum = sums + b * nkv;
  p.q_sum128 = sums + b * nkv + b * (np / 32);
  p.dq = static_cast<uint16_t*>(dq);
  p.dk = static_cast<uint16_t*>(dk);
  p.dv = static_cast<uint16_t*>(dv);
  p.n = n;
  p.np = np;
  p.h = (int)h;
  p.sm_scale = sm_scale;
  // the last dQ items (up to kBwdDqSplit, a multiple of 8) in two key halves
  // (measured at 1x30x4416x128: 1150.6 -> 1124.5 us with 128; 64 and 256
  // within the run-to-run spread of 128)
  const int64_t items = bh * (np / 128);
  p.dq_split = nkv >= 2 && bwd_split_enabled() ? (int)std::min<int64_t>(sage::kBwdDqSplit, items / 8 * 8) : 0;
  p.dq_part = reinterpret_cast<float*>(w + ws.dq_part);
  p.dq_ctr = reinterpret_cast<uint64_t*>(w + ws.dq_ctr);
  p.dq_tag = next_merge_tag();
  return launch_status(sage::launch_bwd(qk_kind, mask, p, d, bh, stream), "sage_attn_bwd");
}

int sage_build_tile_mask(const int32_t* doc_ids, int64_t b, int64_t n, int32_t pad_fill, uint8_t* mask,
                         hipStream_t stream) {
  if (b <= 0 || n <= 0) return fail(SAGE_ERR_ARG, "b=%lld and n=%lld must be positive", (long long)b, (long long)n);
  if (b > 65535) return fail(SAGE_ERR_ARG, "b=%lld exceeds the grid limit 65535", (long long)b);
  if (n > (int64_t)1 << 24) return fail(SAGE_ERR_ARG, "n=%lld exceeds 2^24", (long long)n);
  if (!doc_ids || !mask) return fail(SAGE_ERR_ARG, "null tensor pointer");
  return launch_status(sage::launch_tile_mask(doc_ids, b, n, pad_fill, mask, stream), "sage_build_tile_mask");
}

int sage_doc_ids_from_cu_seqlens(const int32_t* cu_seqlens, int64_t b, int64_t n_segments, int64_t n,
                                 int32_t* doc_ids, hipStream_t stream) {
  if (b <= 0 || n <= 0) return fail(SAGE_ERR_ARG, "b=%lld and n=%lld must be positive", (long long)b, (long long)n);
  if (n_segments < 0) return fail(SAGE_ERR_ARG, "n_segments=%lld must not be negative", (long long)n_segments);
  if (b > 65535) return fail(SAGE_ERR_ARG, "b=%lld exceeds the grid limit 65535", (long long)b);
  if (n > (int64_t)1 << 24) return fail(SAGE_ERR_ARG, "n=%lld exceeds 2^24", (long long)n);
  if (!cu_seqlens || !doc_ids) return fail(SAGE_ERR_ARG, "null tensor pointer");
  return launch_status(sage::launch_doc_from_cu(cu_seqlens, b, n_segments, n, doc_ids, stream),
                       "sage_doc_ids_from_cu_seqlens");
}

}  // extern "C"
