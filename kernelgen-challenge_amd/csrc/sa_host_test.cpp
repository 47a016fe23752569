// sa_host_test.cpp -- g++-only build of the host-side argument validation and
// split-topk planning (sa_plan.h), exported for CPU unit tests. Not part of the
// product ABI; the HIP library compiles the same header.
#include "sa_plan.h"

extern "C" {

int sa_host_validate(const sa_args* a) { return sa::validate(a); }

int sa_host_validate_merge(const sa_merge_args* a) { return sa::validate_merge(a); }

// sa_workspace_bytes with a given CU count: the plan's bytes and, below 16
// heads, the 16-head copy of q and o (sa::pad_layout).
int sa_host_workspace_bytes(const sa_args* a, int num_cus, int64_t* out) {
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  const size_t plan = sa::make_plan(a, num_cus).ws_bytes;
  *out = int64_t(plan + sa::pad_layout(a, plan).bytes);
  return SA_OK;
}

int sa_host_plan(const sa_args* a, int num_cus, int64_t* nsplit, int64_t* split_len,
                 size_t* ws_bytes) {
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  const sa::Plan p = sa::make_plan(a, num_cus);
  *nsplit = p.nsplit;
  *split_len = p.split_len;
  *ws_bytes = p.ws_bytes;
  return SA_OK;
}

// out[0..6] = nsplit, split_len, tiles, tiles_per_b, ntiles, tile_cap, ws_bytes;
// out[7..11] = workspace offsets of the tile meta, tile order, union rows,
// multiplicities and split partials
int sa_host_plan_full(const sa_args* a, int num_cus, int64_t* out) {
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  const sa::Plan p = sa::make_plan(a, num_cus);
  out[0] = p.nsplit;
  out[1] = p.split_len;
  out[2] = p.tiles ? 1 : 0;
  out[3] = p.tiles_per_b;
  out[4] = p.ntiles;
  out[5] = p.tile_cap;
  out[6] = int64_t(p.ws_bytes);
  out[7] = int64_t(p.meta_off);
  out[8] = int64_t(p.order_off);
  out[9] = int64_t(p.rows_off);
  out[10] = int64_t(p.cnts_off);
  out[11] = int64_t(p.part_off);
  return SA_OK;
}

}  // extern "C"
