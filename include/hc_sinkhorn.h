/* hc_sinkhorn.h -- C-ABI of the gfx950 hc_split_sinkhorn kernels (track 02).
 *
 * Replaces the Triton kernels behind the reference entry point
 * track-02/submission.py:316-444 (hc_split_sinkhorn); the arithmetic is
 * track-02/reference/reference.py:38-51. Per token (one row of `mixes`):
 *
 *   pre[k]    = sigmoid(mixes[k]     * scale[0] + base[k])     + eps   k < 4
 *   post[k]   = 2 * sigmoid(mixes[4+k] * scale[1] + base[4+k])         k < 4
 *   comb[i,j] = mixes[8+4i+j] * scale[2] + base[8+4i+j], softmax over j, + eps,
 *               then every column divided by its sum + eps, then
 *               (iters - 1) rounds of: rows divided by their sum + eps, then
 *               columns divided by their sum + eps.
 *
 * All buffers are device memory, fp32, contiguous and 16-byte aligned; the
 * caller owns them. The call is asynchronous on `hip_stream` and allocates
 * nothing. Reentrant; the library keeps no state.
 */
#ifndef HC_SINKHORN_H
#define HC_SINKHORN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HC_ABI_VERSION 1

enum {
  HC_OK = 0,
  HC_EINVAL = 1,        /* null / misaligned pointer, negative size, bad flags */
  HC_EUNSUPPORTED = 2,  /* hc_mult != 4 (as track-02/submission.py:341) or n too large */
  HC_EHIP = 3           /* a HIP launch failed */
};

/* Lanes per token. 16: one matrix entry per lane, sums by DPP within the
 * token's 16 lanes (shortest dependency chain: small n). 1: one token per
 * lane (least work per token: large n). 0 lets the library choose from n. */
enum { HC_FLAG_LANES16 = 1u, HC_FLAG_LANES1 = 2u };

typedef struct hc_args {
  const float* mixes;  /* [n, 24] */
  const float* scale;  /* [3] */
  const float* base;   /* [24] */
  float* pre;          /* [n, 4] */
  float* post;         /* [n, 4] */
  float* comb;         /* [n, 4, 4], row-major per token */
  int64_t n;           /* tokens: b * s of the reference's [b, s, 24] */
  int32_t hc_mult;     /* must be 4 */
  int32_t iters;       /* sinkhorn_iters; below 1 only the first column division runs */
  float eps;
  uint32_t flags;      /* 0, HC_FLAG_LANES16 or HC_FLAG_LANES1 */
} hc_args;

/* HC_ABI_VERSION of the library. */
int hc_abi_version(void);

/* Static description of a return code. */
const char* hc_strerror(int rc);

/* The whole operation, one kernel launch (none when n == 0).
 * Replaces track-02/submission.py:316 (hc_split_sinkhorn) below its
 * allocation of pre / post / comb (:353-355). */
int hc_split_sinkhorn(const hc_args* a, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* HC_SINKHORN_H */
