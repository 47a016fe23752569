// sa_plan.h -- host-side argument validation and launch planning for the
// gfx950 sparse_attn kernels. Plain C++ (no HIP): the same code is compiled
// into the HIP library and into a g++-built host test library.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "sparse_attn.h"

namespace sa {

constexpr int kHeads = 16;        // h the kernels are built for
constexpr int kDim = 512;         // d the kernels are built for
constexpr int kTileRows = 64;     // gathered kv rows per pipeline step
constexpr int64_t kMaxUnits = int64_t(1) << 24;  // work-groups per launch

// Shared-row tiles: kTileQueries consecutive queries of one batch gather the
// union of their rows once. The union is built from a per-row count table in
// LDS (one byte per query, 8 bytes per row), so it needs kv_len <= kMaxTileKv.
constexpr int kTileQueries = 8;
constexpr int64_t kMaxTileKv = 16384;
// The index kernel counts a tile's slots (kTileQueries * topk, plus one round
// of loads past the end) in 32-bit integers: tiles need topk <= 2^27.
constexpr int64_t kMaxTileTopk = int64_t(1) << 27;

// Tile modes written by the index kernel.
constexpr int kModePerQuery = 0;
constexpr int kModeShared = 1;
constexpr int kMetaInts = 4;  // per tile: union size, mode, valid slots, spare

// Launch plan.
//  * per-query kernel: the topk axis of every (b, m) query is cut into
//    `nsplit` contiguous parts of `split_len` slots, one work-group per part,
//    merged by the combine kernel when nsplit > 1;
//  * shared-row path (`tiles`): an index kernel builds each tile's row union,
//    a one-work-group pass orders the tiles by descending step count (longest
//    first, so the last work-groups to start are the short ones), then tiles
//    whose queries overlap enough run in the shared-row kernel, and the
//    queries of the others in a per-query launch after it.
struct Plan {
  int64_t units;       // b * m
  int nsplit;          // parts per query (1 = no combine pass)
  int64_t split_len;   // slots per part
  bool tiles;          // shared-row path enabled
  int64_t tiles_per_b; // ceil(m / kTileQueries)
  int64_t ntiles;      // b * tiles_per_b
  int64_t tile_cap;    // union entries stored per tile (multiple of kTileRows);
                       // each has a 32-bit row offset and kTileQueries fp16
                       // log2 multiplicities
  size_t meta_off, order_off, rows_off, cnts_off, part_off;  // workspace byte offsets
  size_t ws_bytes;     // total workspace
};

// Bytes of partial state per (query, part): running max and sum per head
// (2 * 16 fp32) followed by the unnormalised output (16 * 512 fp32).
constexpr size_t kPartialMLBytes = 2 * kHeads * sizeof(float);
constexpr size_t kPartialOBytes = size_t(kHeads) * kDim * sizeof(float);

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Head counts the library runs. The kernels compute 16 heads at a time (the
// MFMA M dimension); 16 k heads run as k calls on 16-head slices, and 1, 2, 4
// or 8 heads (powers of two, as the reference's kernels take,
// track-01/submission.py:1004, :1233) are padded to 16 in the workspace.
inline bool heads_supported(int64_t h) {
  return h == 1 || h == 2 || h == 4 || h == 8 || (h >= kHeads && h % kHeads == 0);
}

// Workspace of the 16-head copy of a call with fewer heads, after the plan's
// own bytes: q and o as contiguous [b, m, 16, d] bf16, 16 sink entries and,
// with lse, lse as [b, m, 16] fp32. Zero bytes for h >= 16.
struct PadLayout {
  size_t q_off, o_off, sink_off, lse_off, bytes;
};
inline PadLayout pad_layout(const sa_args* a, size_t base) {
  PadLayout l{};
  if (a->h >= kHeads) return l;
  const size_t bm = size_t(a->b) * size_t(a->m);
  const size_t qo = bm * kHeads * kDim * 2;
  l.q_off = round_up(base, 256);
  l.o_off = round_up(l.q_off + qo, 256);
  l.sink_off = round_up(l.o_off + qo, 256);
  l.lse_off = round_up(l.sink_off + kHeads * 4, 256);
  const size_t end = a->lse != nullptr ? l.lse_off + bm * kHeads * 4 : l.lse_off;
  l.bytes = round_up(end, 256) - base;
  return l;
}

// Checks everything that does not need the device. Returns SA_OK or an error.
inline int validate(const sa_args* a) {
  if (a == nullptr) return SA_EINVAL;
  if (a->b < 0 || a->m < 0 || a->h < 0 || a->d < 0 || a->kv_len < 0 ||
      a->topk < 0)
    return SA_EINVAL;
  if (!heads_supported(a->h) || a->d != kDim) return SA_EUNSUPPORTED;
  if ((a->flags & ~uint32_t(SA_FLAG_PER_QUERY | SA_FLAG_FORCE_TILES | SA_FLAG_PLANNED |
                            SA_FLAG_TILE_SKIP | SA_FLAG_TILE_DENSE | SA_FLAG_TILE_ORDERED)) != 0)
    return SA_EINVAL;
  if ((a->flags & SA_FLAG_TILE_SKIP) != 0 && (a->flags & SA_FLAG_TILE_DENSE) != 0)
    return SA_EINVAL;
  if (a->b == 0 || a->m == 0) return SA_OK;  // empty output, nothing to read
  if (a->q == nullptr || a->o == nullptr || a->sink == nullptr)
    return SA_EINVAL;
  if (a->topk > 0 && a->idx == nullptr) return SA_EINVAL;
  if (a->kv_len > 0 && a->kv == nullptr) return SA_EINVAL;
  if (a->kv_len > (int64_t(1) << 31) - 1) return SA_EUNSUPPORTED;
  if (a->topk > (int64_t(1) << 31) - 1) return SA_EUNSUPPORTED;
  // unit inner strides
  if (a->sq[3] != 1 || a->so[3] != 1 || a->skv[2] != 1) return SA_EINVAL;
  if (a->topk > 0 && a->sidx[2] != 1) return SA_EINVAL;
  // 16-byte row loads and stores
  if (!aligned16(a->q) || !aligned16(a->o)) return SA_EINVAL;
  if (a->kv_len > 0 && !aligned16(a->kv)) return SA_EINVAL;
  if (a->workspace != nullptr && !aligned16(a->workspace)) return SA_EINVAL;  // vector loads
  for (int i = 0; i < 3; ++i)
    if (a->sq[i] % 8 != 0 || a->so[i] % 8 != 0) return SA_EINVAL;
  for (int i = 0; i < 2; ++i)
    if (a->skv[i] % 8 != 0) return SA_EINVAL;
  for (int i = 0; i < 3; ++i)
    if (a->sq[i] < 0 || a->so[i] < 0) return SA_EINVAL;
  if (a->skv[0] < 0 || a->skv[1] < 0) return SA_EINVAL;
  if (a->sidx[0] < 0 || a->sidx[1] < 0) return SA_EINVAL;
  if (!(a->scale == a->scale)) return SA_EINVAL;  // NaN scale
  if (a->lse != nullptr) {
    if ((reinterpret_cast<uintptr_t>(a->lse) & 3u) != 0) return SA_EINVAL;
    for (int i = 0; i < 3; ++i)
      if (a->slse[i] < 0) return SA_EINVAL;
  }
  if (a->b > kMaxUnits || a->m > kMaxUnits || a->b * a->m > kMaxUnits)
    return SA_EUNSUPPORTED;
  return SA_OK;
}

// Checks the arguments of sa_merge. Returns SA_OK or an error.
inline int validate_merge(const sa_merge_args* a) {
  if (a == nullptr) return SA_EINVAL;
  if (a->n < 0 || a->b < 0 || a->m < 0 || a->h < 0 || a->d < 0) return SA_EINVAL;
  if (a->b == 0 || a->m == 0 || a->h == 0 || a->d == 0) return SA_OK;  // nothing to write
  if (a->d % 8 != 0) return SA_EINVAL;
  if (a->o == nullptr || !aligned16(a->o) || a->so[3] != 1) return SA_EINVAL;
  for (int i = 0; i < 3; ++i)
    if (a->so[i] < 0 || a->so[i] % 8 != 0) return SA_EINVAL;
  if (a->n > 0) {
    if (a->o_parts == nullptr || a->lse_parts == nullptr) return SA_EINVAL;
    if (!aligned16(a->o_parts) || a->sop[4] != 1) return SA_EINVAL;
    for (int i = 0; i < 4; ++i)
      if (a->sop[i] < 0 || a->sop[i] % 8 != 0 || a->slp[i] < 0) return SA_EINVAL;
    if ((reinterpret_cast<uintptr_t>(a->lse_parts) & 3u) != 0) return SA_EINVAL;
  }
  if (a->lse != nullptr) {
    if ((reinterpret_cast<uintptr_t>(a->lse) & 3u) != 0) return SA_EINVAL;
    for (int i = 0; i < 3; ++i)
      if (a->slse[i] < 0) return SA_EINVAL;
  }
  if (a->sink != nullptr && (reinterpret_cast<uintptr_t>(a->sink) & 3u) != 0) return SA_EINVAL;
  if (a->b > kMaxUnits || a->m > kMaxUnits || a->h > kMaxUnits ||
      a->b * a->m > kMaxUnits * 16 || a->b * a->m * a->h > (int64_t(1) << 31) - 1)
    return SA_EUNSUPPORTED;
  return SA_OK;
}

// Split-topk plan. A query is cut only when there are fewer queries than
// compute units, and never into parts shorter than one pipeline tile, so
// decode shapes (few queries, long topk) still occupy every CU. Shared-row
// tiles are planned when every query has its own work-group (no split), the
// batch has at least half a tile, the count table fits in LDS and the tile's
// slot count fits 32 bits.
inline Plan make_plan(const sa_args* a, int num_cus) {
  Plan p{};
  p.units = a->b * a->m;
  p.nsplit = 1;
  p.split_len = a->topk;
  if (num_cus < 1) num_cus = 1;
  if (p.units > 0 && p.units < num_cus && a->topk > kTileRows) {
    int64_t want = (num_cus + p.units - 1) / p.units;
    int64_t max_parts = (a->topk + kTileRows - 1) / kTileRows;
    if (want > max_parts) want = max_parts;
    if (want > 1) {
      // parts are whole tiles so only the last one has a ragged tail
      int64_t tiles = (a->topk + kTileRows - 1) / kTileRows;
      int64_t tiles_per = (tiles + want - 1) / want;
      p.split_len = tiles_per * kTileRows;
      p.nsplit = int((a->topk + p.split_len - 1) / p.split_len);
    }
  }
  if (p.units * p.nsplit > kMaxUnits) {  // keep the grid launchable
    p.nsplit = 1;
    p.split_len = a->topk;
  }
  // the shared-row kernel addresses rows by 32-bit byte offsets in the batch
  const bool offsets32 =
      a->kv_len > 0 && (a->kv_len - 1) * a->skv[1] * 2 + 2 * kDim <= int64_t(UINT32_MAX);
  p.tiles = p.nsplit == 1 && (a->flags & SA_FLAG_PER_QUERY) == 0 &&
            a->m >= kTileQueries / 2 && a->topk > 0 && a->topk <= kMaxTileTopk &&
            a->kv_len > 0 && a->kv_len <= kMaxTileKv && offsets32;
  size_t off = 0;
  if (p.tiles) {
    p.tiles_per_b = (a->m + kTileQueries - 1) / kTileQueries;
    p.ntiles = a->b * p.tiles_per_b;
    int64_t cap = a->kv_len < kTileQueries * a->topk ? a->kv_len : kTileQueries * a->topk;
    p.tile_cap = int64_t(round_up(size_t(cap), kTileRows));
    p.meta_off = off;
    off = round_up(off + size_t(p.ntiles) * kMetaInts * 4, 256);
    p.order_off = off;
    off = round_up(off + size_t(p.ntiles) * 4, 256);
    p.rows_off = off;
    off = round_up(off + size_t(p.ntiles) * p.tile_cap * 4, 256);
    p.cnts_off = off;  // fp16 log2 multiplicity per (union entry, tile query)
    off = round_up(off + size_t(p.ntiles) * p.tile_cap * kTileQueries * 2, 256);
  }
  if (p.nsplit > 1) {
    p.part_off = off;
    off += size_t(p.units) * p.nsplit * (kPartialMLBytes + kPartialOBytes);
  }
  p.ws_bytes = off;
  return p;
}

}  // namespace sa
