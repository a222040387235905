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
  // [B][Np/128] with document ids, per 128-row query tile: (first scheduled
  // key tile, one past the last scheduled key tile that some live wave of
  // the tile does not see whole (0 if none), one past the last scheduled key
  // tile, 0); an item with no scheduled tile has first = nT, last = 0
  const int4* doc_range;
  // with document ids: [0].x the number of listed split query tiles, [1 + e].x
  // = b * nq + qt of entry e < heavy_max (doc_prefix_kernel); the first
  // heavy_max * h workgroups take them
  int4* heavy;
  int heavy_max;
  uint16_t* out;
  // element strides of out per batch, head and row: [B,H,N,D] is
  // (H*N*D, N*D, D), [B,N,H,D] is (N*H*D, D, H*D)
  int64_t out_bs, out_hs, out_rs;
  float* lse;
  int64_t n;
  int64_t np;
  int h;           // heads per batch
  int bh;          // B * H
  int nt;          // key tiles: ceil(N / 64)
  int light_last;  // last 128-row query tile holds <= 64 rows: schedule those items last
  // unmasked launches: the items past n_whole (in schedule order) are cut into
  // split_parts key-tile ranges whose partials a second kernel merges
  int n_whole;
  int split_parts;
  float* part;  // (items - n_whole) * split_parts slots of kPartFloats<D> floats
  // in-kernel merge: one arrival counter per split item (the last piece to
  // arrive merges the item); null: merge_split_kernel merges after the launch.
  // A counter holds merge_tag << 8 | pieces arrived; the merging piece resets
  // it to merge_tag << 8, so a graph replay with the same tag counts from 0.
  uint64_t* merge_ctr;
  uint64_t merge_tag;
  // parity only (int8 QK, unmasked): int32 [BH, Np, Np] receives the S^T
  // accumulators of every tile the kernel's own loop consumes (row = query)
  int32_t* s_dump;
};

// Split query tiles (document ids) that the first workgroups of a launch take
// (AttnParams::heavy): kHeavyMax * h workgroups are reserved for them.
constexpr int kHeavyMax = 2;

// Resident workgroups of the attention kernel on MI355X: 256 CUs x 2.
constexpr int kResidentWGs = 512;

// Floats of one partial slot: O of 128 rows x D (fp32, lane order), then the
// per-lane reference point and row-sum halves of the 4 waves.
template <int D>
constexpr int64_t kPartFloats = 128 * D + 2 * 256;

// Tail split of an unmasked launch of n_items 128-row items of nt key tiles:
// whole items fill complete rounds of the resident workgroups; the items of
// the last, partial round are cut into `parts` ranges of key tiles (at most
// 4), chosen to minimize (rounds the pieces take) x (tiles per piece + 2
// tiles of pipeline start).  The cap of 4 is measured: at 1050 items of 69
// tiles, 4 pieces beat 8 (257.6 vs 260.0 us) and 2 (271.7 us), since the
// partials' traffic and merge grow with the piece count and the pieces run
// beside the second round's last items.
//
// Launches of less than one round: an item alone on a CU runs about 1.4x
// faster than one of two sharing it (its waves have the SIMDs' issue slots to
// themselves), so when up to 128 items spill past one per CU, the first 256
// stay whole and the spilled items are cut into key-tile pieces that share
// the CUs with them: 4 pieces (at least 2 tiles each) while every piece still
// fits the one round of resident workgroups, else as many as fit, at least 2.
// Measured at 20 tiles with a separate merge kernel: 2 pieces, 260 items
// 43.5 -> 34.8 us, 300 items 41.6 -> 36.9, 350 items 41.5 -> 39.1; 400 items
// lose, 42.1 -> 55.7; cutting every item costs more than it balances (300
// items: 54.3 / 57.7 / 59.6 us in 2 / 3 / 4 pieces).  With the merge inside
// the attention kernel, 300 items: 34.4 us in 2 pieces, 31.7 / 31.6 in 3 / 4,
// 33.1 in 5.
struct TailSplit {
  int64_t whole;
  int parts;
};

inline TailSplit tail_split(int64_t n_items, int64_t nt) {
  TailSplit t{n_items, 1};
  constexpr int64_t kCUs = kResidentWGs / 2;
  if (n_items > kCUs && n_items < kResidentWGs) {
    const int64_t spill = n_items - kCUs;
    if (spill <= 128 && nt >= 2) {
      int64_t parts = kCUs / spill;  // pieces that fit the round
      parts = parts < 4 ? parts : 4;
      parts = parts < nt / 2 ? parts : nt / 2;
      t = TailSplit{kCUs, (int)(parts > 2 ? parts : 2)};
    }
    return t;
  }
  const int64_t rest = n_items >= kResidentWGs ? n_items % kResidentWGs : 0;
  if (rest == 0) return t;
  int64_t best = (rest + kResidentWGs - 1) / kResidentWGs * (nt + 2);
  const int pmax = (int)(nt < 4 ? nt : 4);
  for (int p = 2; p <= pmax; ++p) {
    const int64_t cost = (rest * p + kResidentWGs - 1) / kResidentWGs * ((nt + p - 1) / p + 2);
    if (cost < best) {
      best = cost;
      t.parts = p;
    }
  }
  if (t.parts > 1) t.whole = n_items - rest;
  return t;
}

// Inputs of the q/k/v producer (QKV split + per-head RMSNorm + Flux RoPE +
// transpose, fused_kernels.py:271-390).  With qkv set, the quantization reads
// the projection output and applies the producer itself; with qkv null it
// reads bf16 q, k, v [BH, N, D].
// Heads per slab unit of the producer kernels (one pass of tokens for this
// many heads of a batch in one workgroup).
constexpr int kSlabHeads = 8;

struct ProdArgs {
  const uint16_t* qkv;  // bf16 [B, N, 3*H*D]
  const float* qw;      // RMSNorm weights of q and k, fp32 [D]
  const float* kw;
  const float* freqs;   // fp32 [B*N, D/2, 2, 2]: [[cos, -sin], [sin, cos]] per channel pair
  int h;
  int bh;               // B*H
  float eps;
};

hipError_t launch_quantize(int qk, int pv, int gran, bool smooth, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, int64_t bh, int64_t n, int64_t d, float fold, double* ws,
                           uint8_t* qc, float* qs, uint8_t* kc, float* ks, uint8_t* vout, float* vs,
                           uint16_t* kmean, const ProdArgs& prod, hipStream_t st);
hipError_t launch_qkv_postprocess(const ProdArgs& prod, int64_t bh, int64_t n, int64_t d, uint16_t* q_out,
                                  uint16_t* k_out, uint16_t* v_out, hipStream_t st);
// Gradient of the producer with respect to its input (fused_kernels.py:711-783):
// gq, gk, gv bf16 [BH, N, D] -> dqkv bf16 [B, N, 3*H*D].
hipError_t launch_qkv_postprocess_bwd(const ProdArgs& prod, int64_t bh, int64_t n, int64_t d, const uint16_t* gq,
                                      const uint16_t* gk, const uint16_t* gv, uint16_t* dqkv, hipStream_t st);
size_t quant_workspace_bytes(int64_t bh, int64_t n, int64_t d);
int64_t quant_grid_units(int64_t bh, int64_t n, int64_t d, int64_t h_producer);

hipError_t launch_attn(int qk, int pv, int gran, int mask, const AttnParams& p, int64_t d, int nb, hipStream_t st);
// Per-batch document-id summaries (min doc, max doc, #valid, #padding) of every
// 64-key tile ([nb][ceil(n/64)]), 32-row block ([nb][Np/32]) and 128-row block
// ([nb][Np/128]).
// The scheduled key-tile range of each 128-row query tile and one past the
// last key tile that some live wave of it does not see whole (the doc_range
// entries), from the summaries (after launch_doc_summaries).
// Also lists the query tiles whose live waves see different key-tile ranges
// (heavy, when not null; see AttnParams::heavy).
hipError_t launch_doc_prefix(const int4* kv_sum, const int4* q_sum, const int4* q_sum128, int64_t n, int nb,
                             int4* range, int4* heavy, hipStream_t st);
// heavy (may be null): the split-query-tile list to empty before launch_doc_prefix.
hipError_t launch_doc_summaries(const int32_t* doc, int64_t n, int nb, int4* kv_sum, int4* q_sum, int4* q_sum128,
                                int4* heavy, hipStream_t st);
// Workspace of one attention call: the doc-id summaries, then the partial
// slots of the tail split.
struct AttnWorkspace {
  size_t doc_off, heavy_off, part_off, ctr_off, bytes;
  TailSplit split;
};
// `masked`: a launch with a tile mask or document ids, which splits no item
// and so needs no partial slots
AttnWorkspace attn_workspace(int64_t b, int64_t h, int64_t n, int64_t d, bool masked = false);
size_t attn_workspace_bytes(int64_t b, int64_t h, int64_t n, int64_t d, bool masked = false);
hipError_t launch_tile_mask(const int32_t* doc, int64_t nb, int64_t n, int32_t pad_fill, uint8_t* mask,
                            hipStream_t st);

// Backward (sage_kernels.py:321-349, :805-1030, :1491-1722).  Codes and
// scales are the quantization's per-token outputs ([BH, Np] layout, Q scale
// with sm_scale*log2(e)); tq / tk / tdo are T images [BH, Np, D] of Q, the
// smoothed K and dO, rdo / rv R images of dO and V; v, dout, lse and the
// gradients are unpadded [BH, N(, D)]; delta is [BH, Np].
struct BwdParams {
  const uint8_t* qc;
  const float* qs;
  const uint8_t* kc;
  const float* ks;
  const uint16_t* v;
  const uint16_t* dout;
  const uint16_t* tq;
  const uint16_t* tk;
  const uint16_t* tdo;
  const uint16_t* rdo;  // R images [BH, Np, D] of dO and V
  const uint16_t* rv;
  const float* lse;
  const float* delta;
  const uint8_t* tile_mask;
  int64_t mask_stride_z;
  int64_t mask_nkv;
  const int32_t* doc;     // [B, N] document ids (mask bit 2)
  const int4* kv_sum;     // their summaries: [B][ceil(N/64)] key tiles,
  const int4* q_sum;      // [B][Np/32] and [B][Np/128] query blocks
  const int4* q_sum128;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t n, np;
  int h;
  float sm_scale;
  // the last dq_split dQ items of the launch (a multiple of 8) run as two
  // key-tile halves, dispatched last: fp32 partial dQ slots [dq_split][2]
  // of 128 * D floats, one arrival counter per cut item (dq_tag << 8 | halves
  // arrived; the merging half resets it to dq_tag << 8)
  int dq_split;
  float* dq_part;
  uint64_t* dq_ctr;
  uint64_t dq_tag;
};

// dQ items of a backward launch cut in two key-tile halves (at most; a
// multiple of 8, so both halves of an item run on one XCD).
constexpr int kBwdDqSplit = 64;

// Two operand-image jobs of one launch: x [BH, N, D] bf16 -> out [BH, Np, D]
// (T or R image), with mu ([BH, D] bf16) subtracted when set (T images only).
struct TImageJobs {
  const uint16_t* x[2];
  const uint16_t* mu[2];
  uint16_t* out[2];
};

hipError_t launch_bwd_prep(const TImageJobs& tjobs, const TImageJobs& rjobs, const uint16_t* dout,
                           const uint16_t* out, int64_t bh, int64_t n, int64_t d, float* delta, hipStream_t st);
hipError_t launch_bwd(int qk, int mask, const BwdParams& p, int64_t d, int64_t bh, hipStream_t st);
hipError_t launch_doc_from_cu(const int32_t* cu, int64_t nb, int64_t nseg, int64_t n, int32_t* doc,
                              hipStream_t st);

}  // namespace sage
