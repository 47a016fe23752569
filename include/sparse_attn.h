/*
 * sparse_attn.h -- C-ABI of the MI355X (gfx950) sparse_attn hot path.
 *
 * The op: for every (batch b, query m, head h)
 *
 *   o[b,m,h,:] = sum_t softmax([s_0 .. s_{topk-1}, sink[h]])_t * kv[b, idx[b,m,t], :]
 *   s_t        = scale * <q[b,m,h,:], kv[b, idx[b,m,t], :]>
 *
 * with the sink's own column dropped from the weighted sum. This is the
 * reference oracle track-01/reference/reference.py:24-40 and the argument
 * contract of track-01/requirements.md:92-114 (q, kv bf16; attn_sink fp32 per
 * head; topk_idxs int32; o bf16 in q's layout).
 *
 * Index values:
 *   -1                 padding sentinel: the slot is excluded (score -inf,
 *                      its row is never read), as the sentinel handling of
 *                      track-01/submission.py:313-322. A row whose slots are
 *                      all -1 yields o = 0 (the sink takes all the mass).
 *   0 .. kv_len-1      valid; duplicates count with multiplicity.
 *   anything else      out of range: the slot is excluded, never read, and
 *                      1 is stored into *err_word (if non-null). The reference
 *                      raises here (torch.gather at reference.py:28); the
 *                      Python layer turns the flag into RuntimeError.
 *
 * Shapes (ABI version 7): d = 512; h = 1, 2, 4, 8 or a multiple of 16 (the
 * reference's kernels take power-of-two h, track-01/submission.py:1004,
 * :1233; the contest fixes h = 16). The kernels compute 16 heads at a time:
 * 16 k heads run as k passes over 16-head slices, and fewer heads on a
 * zero-padded 16-head copy in the workspace (sa_workspace_bytes counts it).
 *
 * Threading and ownership: the caller owns every buffer. The library keeps no
 * mutable state apart from a per-device cache of the compute-unit count, and
 * every entry point is reentrant. sa_forward is asynchronous on the given
 * HIP stream.
 */
#ifndef SPARSE_ATTN_H
#define SPARSE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_ABI_VERSION 9

/* Return codes. */
enum {
  SA_OK = 0,
  SA_EINVAL = 1,        /* null pointer, negative size, bad stride or alignment */
  SA_EUNSUPPORTED = 2,  /* h not 1, 2, 4, 8 or a multiple of 16; d != 512; or a
                           grid beyond the launch limit */
  SA_EWORKSPACE = 3,    /* workspace missing or smaller than sa_workspace_bytes */
  SA_EHIP = 4,          /* HIP runtime error (device query or launch) */
  SA_ESCRATCH = 5       /* (ABI version 4) sa_forward_noalloc: the call needs more
                           than SA_NOALLOC_SCRATCH_BYTES of workspace */
};

/* sa_args.flags bits (0 = let the library choose). */
enum {
  /* every query gathers its own rows (no shared-row tiles) */
  SA_FLAG_PER_QUERY = 1u,
  /* run every eligible tile of consecutive queries through the shared-row
     kernel, whatever the overlap of their indices */
  SA_FLAG_FORCE_TILES = 2u,
  /* (ABI version 3) the workspace holds the index plan of these arguments,
     made by sa_plan_indices: the index-dependent kernels are skipped */
  SA_FLAG_PLANNED = 4u,
  /* (ABI version 7) the form of the shared-row kernel's step. By default the
     pair-skipping form runs when 8 * topk < kv_len (a row is then named by
     fewer than one query of a tile on average, so query pairs often name no
     row of a 32-row half-step and skip its P . V), the dense form otherwise.
     These force one form; both give the same results. Not both at once. */
  SA_FLAG_TILE_SKIP = 8u,
  SA_FLAG_TILE_DENSE = 16u,
  /* (ABI version 9) tile plans with topk <= 384 (per-query queries run as
     WAVE): run the shared-row tiles from the tile order, one work-group per
     tile, after an ORDER launch (none with SA_FLAG_PLANNED), instead of the
     default TILE launch of one work-group per CU that walks the tiles' modes
     and runs the shared ones. Same results. */
  SA_FLAG_TILE_ORDERED = 32u
};

/*
 * Arguments of one call. Strides are in elements. The innermost stride of q,
 * kv and o (d) and of topk_idxs (topk) must be 1; q, kv and o must be 16-byte
 * aligned with their other strides multiples of 8 elements.
 */
typedef struct sa_args {
  const void* q;          /* bf16 [b, m, h, d]                            */
  const void* kv;         /* bf16 [b, kv_len, d]  (K and V share rows)     */
  const float* sink;      /* fp32 [h]                                      */
  const int32_t* idx;     /* int32 [b, m, topk]                            */
  void* o;                /* bf16 [b, m, h, d]  (written)                  */
  int64_t b, m, h, d, kv_len, topk;
  int64_t sq[4];          /* strides of q   */
  int64_t skv[3];         /* strides of kv  */
  int64_t sidx[3];        /* strides of idx */
  int64_t so[4];          /* strides of o   */
  float scale;            /* softmax scale, e.g. d**-0.5 */
  void* workspace;        /* device scratch: tile row unions, split partials;
                             16-byte aligned (ABI version 7) */
  size_t workspace_bytes;
  int32_t* err_word;      /* int32, nullable; set to 1 when a bad index is seen
                             (a system-scope store, never cleared by the library:
                             device memory, or mapped pinned host memory that the
                             host reads without synchronizing) */
  uint32_t flags;         /* SA_FLAG_* bits, normally 0 */
  float* lse;             /* fp32 [b, m, h], nullable: log-sum-exp per (query, head) */
  int64_t slse[3];        /* strides of lse */
} sa_args;

/*
 * lse (when sa_args.lse is set): for each (b, m, h), in natural log,
 *
 *   lse = ln( sum_t exp(s_t) + exp(sink[h]) )
 *
 * over the valid slots, so that o = sum_t exp(s_t - lse) * kv[idx_t]. This is
 * m_total + ln(l_total) of the reference kernel's sink fold
 * (track-01/submission.py:195-199, notes.md:32-41). A query with no mass at
 * all (no valid slot and sink = -inf) gets o = 0 and lse = -inf.
 *
 * Version 2 added lse / slse at the end of sa_args and sa_merge.
 */

/* Version of this ABI (SA_ABI_VERSION). */
int sa_abi_version(void);

/*
 * Bytes of device workspace sa_forward needs for these arguments on the
 * current HIP device: the row unions of shared-row tiles and the partial
 * states of split-topk parts (0 when neither is planned). No counterpart
 * in the reference: its Triton kernels keep all state on chip
 * (track-01/submission.py:143-202); the output allocation it does replace
 * is track-01/submission.py:1000.
 */
int sa_workspace_bytes(const sa_args* a, size_t* out_bytes);

/*
 * Run sparse attention on `hip_stream` (a hipStream_t; NULL = default
 * stream). Replaces the body of sparse_attn in
 * track-01/submission.py:975-1271 (argument unpacking :989-998, the launch
 * of _sparse_attn_kernel_bf16 / _universal at :1005-1021 and :1225-1271).
 * Argument errors return before any device work.
 */
int sa_forward(const sa_args* a, void* hip_stream);

/*
 * Merge of partial results: parts i = 0..n-1 hold attention over disjoint
 * subsets of a query's slots (for example KV shards), each computed with
 * sink = -inf and returned with its lse. The merge folds the sink once:
 *
 *   lse = ln( sum_i exp(lse_i) + exp(sink[h]) )
 *   o   = sum_i exp(lse_i - lse) * o_i
 *
 * which equals sa_forward over the union of the parts' slots (the split-topk
 * combine of this library, exposed as its own op; the sink algebra of
 * track-01/notes.md:32-41). A part with lse_i = -inf contributes nothing.
 * No counterpart in the reference, which always runs the whole top-k in one
 * kernel.
 */
typedef struct sa_merge_args {
  const void* o_parts;     /* bf16 [n, b, m, h, d] */
  const float* lse_parts;  /* fp32 [n, b, m, h]    */
  const float* sink;       /* fp32 [h], nullable (= -inf: no sink) */
  void* o;                 /* bf16 [b, m, h, d]  (written) */
  float* lse;              /* fp32 [b, m, h], nullable (written) */
  int64_t n, b, m, h, d;
  int64_t sop[5];          /* strides of o_parts   */
  int64_t slp[4];          /* strides of lse_parts */
  int64_t so[4];           /* strides of o         */
  int64_t slse[3];         /* strides of lse       */
} sa_merge_args;

/*
 * Run the merge on `hip_stream`. d must be a multiple of 8 with unit stride;
 * o_parts and o 16-byte aligned with their other strides multiples of 8.
 * n = 0 writes o = 0 and lse = sink (or -inf). Asynchronous; argument errors
 * return before any device work.
 */
int sa_merge(const sa_merge_args* a, void* hip_stream);

/*
 * Index preprocessing on its own (ABI version 3). Runs the index-dependent
 * part of sa_forward into a->workspace (sa_workspace_bytes of the same
 * arguments): for a shared-row plan, the validation of every index
 * (*err_word), each 8-query tile's row union and multiplicities and the
 * longest-first tile order; for other plans nothing (their validation and
 * compaction run inside the forward kernel). sa_forward with
 * SA_FLAG_PLANNED and that workspace then starts at the attention kernel,
 * so one plan serves every call that uses the same indices (for example
 * layers that share a top-k selection).
 * The plan depends on the values of topk_idxs and on b, m, kv_len, topk,
 * the index strides, kv's row stride skv[1] and the other flags; q, kv's
 * data, attn_sink, o and lse may differ between the calls. The forward
 * only reads the workspace. No counterpart in the reference, which handles
 * its indices inside each kernel call (track-01/submission.py:177-180,
 * :313-322). Asynchronous; argument errors return before any device work.
 */
int sa_plan_indices(const sa_args* a, void* hip_stream);

/*
 * The allocation-free forward sa_forward_noalloc (ABI version 4) is declared
 * in sparse_attn_noalloc.h and exported by its own library since version 7
 * (see there); SA_ESCRATCH is its return code.
 */

/*
 * Kernels of one sa_forward call. Launch order: per-query plans QUERY, then
 * COMBINE when split; shared-row (tile) plans INDEX (unless SA_FLAG_PLANNED),
 * QUERY, TILE. In a tile plan the QUERY launch runs the queries of the tiles
 * the index kernel made per query, and makes the longest-first tile order
 * in its first work-group. (Version 5: the order no longer had a launch of
 * its own.) Version 6: unsplit plans with topk <= 384 run their per-query
 * queries as WAVE instead, one wave per query. Version 8: where QUERY would
 * only make the tile order (such a plan, and sa_plan_indices), the order is
 * ORDER, a one-work-group launch of its own. Version 9: such a plan makes no
 * order (INDEX, WAVE, TILE; its TILE launch finds the shared tiles itself)
 * unless SA_FLAG_TILE_ORDERED asks for INDEX, ORDER, WAVE, TILE;
 * sa_plan_indices still makes it (INDEX, ORDER).
 */
enum {
  SA_KERNEL_INDEX = 0,    /* row unions of shared-row tiles (tile plans)   */
  SA_KERNEL_ORDER = 1,    /* the tile order alone (versions 8, 9; above)   */
  SA_KERNEL_TILE = 2,     /* shared-row tiles (tile plans)                 */
  SA_KERNEL_QUERY = 3,    /* per-query parts; in tile plans the per-query
                             tiles and the tile order                      */
  SA_KERNEL_COMBINE = 4,  /* merge of split-topk parts (split plans)       */
  SA_KERNEL_WAVE = 5,     /* short unsplit queries, one wave per query     */
  SA_KERNEL_COUNT = 6
};

/*
 * Measurement hook. No counterpart in the reference, which times whole calls
 * from Python (track-01/bench.py:20-47). Same as sa_forward, but kernel k is
 * launched through hipExtLaunchKernel with events[2k] and events[2k + 1] as
 * its start and stop events, which take the dispatch's own start and end
 * timestamps (version 7; before, events recorded on the stream around the
 * launch, which also timed the gap before the dispatch). `events` holds
 * 2 * SA_KERNEL_COUNT of the caller's hipEvent_t handles (created, with
 * timing enabled; a kernel whose two entries are NULL launches without
 * events). Bit k of *launched (if non-null) is set when kernel k was
 * launched. Nothing synchronizes: read the events once the stream has
 * drained.
 */
int sa_forward_events(const sa_args* a, void* hip_stream, void* const* events,
                      uint32_t* launched);

/* Static description of a return code. */
const char* sa_strerror(int code);

#ifdef __cplusplus
}
#endif

#endif /* SPARSE_ATTN_H */
