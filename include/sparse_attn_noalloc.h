/*
 * Allocation-free sparse-attention forward, exported by
 * lib/libsa_noalloc_gfx950.so (which links lib/libsparse_attn_gfx950.so).
 *
 * No counterpart in the reference (track-01/submission.py:975-1000 allocates
 * through torch): it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 *
 * sa_forward_noalloc takes sa_forward's arguments (sparse_attn.h) and runs
 * sa_forward's launches, with the workspace in this library's own file-scope
 * device array of SA_NOALLOC_SCRATCH_BYTES; a->workspace and
 * a->workspace_bytes are ignored. It calls no allocating routine.
 *
 * Footprint: the array is part of this library's code object, so a process
 * that loads the library holds SA_NOALLOC_SCRATCH_BYTES on every GPU it uses
 * the library on, until it ends, whether or not it calls the entry point.
 * Callers of sa_forward alone do not load this library and do not pay it.
 *
 * Limits and errors:
 *  - a call whose sa_workspace_bytes exceeds SA_NOALLOC_SCRATCH_BYTES returns
 *    SA_ESCRATCH before any device work (the five configurations of the
 *    contest's hot path need at most ~40 MiB);
 *  - SA_FLAG_PLANNED is refused (SA_EINVAL): an index plan lives in a
 *    caller's workspace;
 *  - otherwise the return codes of sa_forward.
 *
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents: calls that overlap on one GPU (other streams, other threads)
 * race, so serialize them. Nothing in the array has to start at zero; each
 * call writes what it reads before reading it.
 */
#ifndef SPARSE_ATTN_NOALLOC_H
#define SPARSE_ATTN_NOALLOC_H

#include "sparse_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SA_NOALLOC_SCRATCH_BYTES (48u << 20)

int sa_forward_noalloc(const sa_args* a, void* hip_stream);

/* SA_NOALLOC_SCRATCH_BYTES as this library was built with it. */
int sa_noalloc_scratch_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* SPARSE_ATTN_NOALLOC_H */
