// On-device mask plumbing for packed (multi-document) sequences.
//
// Reference semantics (sqcu/futudiffu):
//   tile mask   src_ii/block_mask.py:84-97: Q tiles of 128 and KV tiles of 64
//               tokens each take the document id of their first token (tile
//               starts clamped to N-1); mask = equality of those ids.  Tokens
//               past the last segment count as document 0 (:75-79).
//   doc ids     src_ii/transformer.py:137-153 (segment i -> id i) and
//               src_ii/forward_packed.py:56-62 (padding to a fixed length
//               with id -1).
// The reference builds the mask on the host with a Python loop over segments;
// here both the mask and the exact per-token ids come from device data
// (document ids or varlen segment offsets), with no host synchronization.
#include "sage_common.h"
#include "sage_launch.h"

namespace sage {

// One thread per (batch, tile pair).  doc is [nb][n]; mask is [nb][nq][nkv].
__global__ void __launch_bounds__(256) tile_mask_kernel(const int32_t* __restrict__ doc, int64_t n, int64_t nq,
                                                        int64_t nkv, int32_t pad_fill, uint8_t* __restrict__ mask) {
  const int64_t pairs = nq * nkv;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pairs) return;
  const int64_t b = blockIdx.y;
  const int64_t i = idx / nkv, j = idx % nkv;
  const int64_t qs = min(i * kRowsPerWG, n - 1), ks = min(j * 64, n - 1);
  int dq = doc[b * n + qs], dk = doc[b * n + ks];
  if (dq < 0) dq = pad_fill;
  if (dk < 0) dk = pad_fill;
  mask[b * pairs + idx] = dq == dk ? 1 : 0;
}

// One thread per (batch, token).  cu is [nb][nseg + 1], nondecreasing per
// batch; token t of batch b gets the segment s with cu[s] <= t < cu[s+1], or
// -1.  Binary search for the last s < nseg with cu[s] <= t: every index read
// stays in [0, nseg] whatever the offsets hold.
__global__ void __launch_bounds__(256) doc_from_cu_kernel(const int32_t* __restrict__ cu, int64_t nseg, int64_t n,
                                                          int32_t* __restrict__ doc) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const int64_t b = blockIdx.y;
  const int32_t* c = cu + b * (nseg + 1);
  int64_t lo = 0, hi = nseg;  // answer in [lo, hi): last s with c[s] <= t, or none
  if (nseg == 0 || (int64_t)c[0] > t) {
    doc[b * n + t] = -1;
    return;
  }
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)c[mid] <= t)
      lo = mid;
    else
      hi = mid;
  }
  doc[b * n + t] = t < (int64_t)c[lo + 1] ? (int32_t)lo : -1;
}

hipError_t launch_tile_mask(const int32_t* doc, int64_t nb, int64_t n, int32_t pad_fill, uint8_t* mask,
                            hipStream_t st) {
  const int64_t nq = (n + kRowsPerWG - 1) / kRowsPerWG, nkv = (n + 63) / 64;
  const int64_t pairs = nq * nkv;
  hipLaunchKernelGGL(tile_mask_kernel, dim3((unsigned)((pairs + 255) / 256), (unsigned)nb), dim3(256), 0, st, doc,
                     n, nq, nkv, pad_fill, mask);
  return hipGetLastError();
}

hipError_t launch_doc_from_cu(const int32_t* cu, int64_t nb, int64_t nseg, int64_t n, int32_t* doc,
                              hipStream_t st) {
  hipLaunchKernelGGL(doc_from_cu_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)nb), dim3(256), 0, st, cu,
                     nseg, n, doc);
  return hipGetLastError();
}

}  // namespace sage
