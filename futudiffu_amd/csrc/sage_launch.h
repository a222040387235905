// Host-side launcher declarations shared by the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sage {

struct AttnParams {
  const uint8_t* qc;
  const float* qs;
  const uint8_t* kc;
  const float* ks;
  const uint8_t* vin;
  const float* vs;
  const uint8_t* tile_mask;
  int64_t mask_stride_z;
  int64_t mask_nkv;
  const int32_t* doc;
  const int4* kv_sum;  // [B][nT]   (min doc, max doc, #valid, #padding) over keys < N
  const int4* q_sum;     // [B][Np/32] same over queries < N
  const int4* q_sum128;  // [B][Np/128] same over queries < N
  uint16_t* out;
  float* lse;
  int64_t n;
  int64_t np;
  int h;           // heads per batch
  int bh;          // B * H
  int nt;          // key tiles: ceil(N / 64)
  int light_last;  // last 128-row query tile holds <= 64 rows: schedule those items last
};

hipError_t launch_quantize(int qk, int pv, int gran, bool smooth, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, int64_t bh, int64_t n, int64_t d, float fold, double* ws,
                           uint8_t* qc, float* qs, uint8_t* kc, float* ks, uint8_t* vout, float* vs,
                           uint16_t* kmean, hipStream_t st);
size_t quant_workspace_bytes(int64_t bh, int64_t n, int64_t d);

hipError_t launch_attn(int qk, int pv, int gran, int mask, const AttnParams& p, int64_t d, int nb, hipStream_t st);
// Workspace of one attention call: the doc-id summaries.
struct AttnWorkspace {
  size_t doc_off, bytes;
};
AttnWorkspace attn_workspace(int64_t b, int64_t h, int64_t n, int64_t d);
size_t attn_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d);
hipError_t launch_qk_int32(const uint8_t* qc, const uint8_t* kc, int64_t bh, int64_t n, int64_t d, int32_t* s,
                           hipStream_t st);

}  // namespace sage
