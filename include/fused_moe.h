/*
 * fused_moe.h -- C-ABI of the MI355X (gfx950) fused mixture-of-experts op
 * (track 03 of the reference).
 *
 * The op, for every token t (track-03/reference/reference.py:10-35):
 *
 *   p      = softmax(score[t, :])                 (fp32)
 *   S      = the topk experts of largest p        (lower index first on ties)
 *   w_e    = bf16(p_e)   or, with renormalize, bf16(p_e / sum_{S} p)
 *   x      = bf16(hidden[t] . w1[e]^T)            [2N]; gate = x[:N], up = x[N:]
 *   u      = bf16(up * bf16(silu(gate)))          [N]
 *   y_e    = bf16(u . w2[e]^T)                    [K]
 *   out[t] = bf16 running sum over e in S, ascending, of bf16(y_e * w_e)
 *
 * Every "bf16(...)" is a round to nearest even, at the points where the
 * reference's bf16 tensors round. The reference leaves ties in the top-k to
 * torch.topk; this library takes the lower expert index first.
 *
 * Ownership and threading: the caller owns every buffer, including the
 * device workspace; the library keeps no mutable state apart from cached
 * device attributes, and every entry point is reentrant. fm_forward is
 * asynchronous on the given HIP stream.
 */
#ifndef FUSED_MOE_H
#define FUSED_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FM_ABI_VERSION 4

enum {
  FM_OK = 0,
  FM_EINVAL = 1,        /* null pointer, negative size, bad stride or alignment */
  FM_EUNSUPPORTED = 2,  /* K % 256, N % 128, E > 256, topk > 32 or sizes past 32-bit offsets */
  FM_EWORKSPACE = 3,    /* workspace missing or smaller than fm_workspace_bytes */
  FM_EHIP = 4           /* HIP runtime error */
};

/* fm_args.flags (0 = let the library choose). */
enum {
  FM_FLAG_LARGE_TILES = 1u,  /* 128-pair tiles whatever the tokens per expert */
  FM_FLAG_SMALL_TILES = 2u,  /* 16-pair weight-streaming tiles */
  FM_FLAG_BIG_TILES = 4u,    /* (ABI version 2) 256-pair tiles, 8 waves per work-group;
                                by default once experts average 256 pairs */
  FM_FLAG_ORDERED_SUM = 8u   /* (ABI version 4) the final sum over a token's experts
                                always runs as its own launch (the ascending-expert
                                running bf16 sum), never as the down GEMM's bf16
                                atomic adds into the output (topk <= 2 with
                                streamed tiles); the result is the same bits.
                                Combines with one tile flag. */
};

typedef struct fm_args {
  const void* hidden;   /* bf16 [M, K], row stride s_hidden, unit inner stride */
  const void* w1;       /* bf16 [E, 2N, K] contiguous (gate rows 0..N-1, up rows N..2N-1) */
  const void* w2;       /* bf16 [E, K, N] contiguous */
  const void* score;    /* bf16 [M, E], row stride s_score, unit inner stride */
  void* out;            /* bf16 [M, K], row stride s_out (written) */
  int64_t M, K, N, E, topk;
  int64_t s_hidden, s_score, s_out;  /* row strides in elements */
  int32_t renormalize;  /* nonzero: the selected weights are divided by their sum */
  uint32_t flags;       /* FM_FLAG_* */
  void* workspace;      /* device scratch of fm_workspace_bytes */
  size_t workspace_bytes;
} fm_args;

int fm_abi_version(void);

/* Bytes of device workspace fm_forward needs for these arguments: routing
   (ids, weights), the pairs sorted by expert, the tile table, the gated
   intermediate [M*topk, N] and the weighted expert outputs [M*topk, K]
   (bf16). No counterpart in the reference, whose torch oracle allocates
   its intermediates per expert (reference.py:28-35). */
int fm_workspace_bytes(const fm_args* a, size_t* out_bytes);

/* Run the op on `hip_stream` (NULL = default stream). Replaces
   fused_moe in track-03/submission.py (its Triton route / gate-up / down
   kernels) and the oracle's loop, reference.py:10-35. Argument errors
   return before any device work. */
int fm_forward(const fm_args* a, void* hip_stream);

/* Kernels of one fm_forward call, in launch order. */
enum {
  FM_KERNEL_ROUTE = 0,   /* softmax + top-k per token                */
  FM_KERNEL_PLAN = 1,    /* pairs sorted by expert, tile table       */
  FM_KERNEL_GATEUP = 2,  /* x = h . w1^T, u = up * silu(gate)        */
  FM_KERNEL_DOWN = 3,    /* y = u . w2^T, times the routing weight   */
  FM_KERNEL_REDUCE = 4,  /* ascending-expert bf16 sum per token; since
                            version 3 not launched for topk <= 2 with
                            streamed (decode) tiles: the down GEMM adds
                            into out itself                          */
  FM_KERNEL_COUNT = 5
};

/* Measurement hook (no counterpart in the reference): fm_forward that
   launches kernel k through hipExtLaunchKernel with events[2k] /
   events[2k + 1] (created hipEvent_t with timing; a kernel whose two entries
   are NULL launches without events) as its start and stop events, which take
   the dispatch's own start and end timestamps (ABI version 4; before, events
   recorded on the stream around the launch), and sets bit k of *launched. */
int fm_forward_events(const fm_args* a, void* hip_stream, void* const* events,
                      uint32_t* launched);

const char* fm_strerror(int code);

#ifdef __cplusplus
}
#endif

#endif /* FUSED_MOE_H */
