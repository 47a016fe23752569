// fused_moe_gfx950.hip -- MI355X (gfx950, CDNA4) kernels and C-ABI of the
// fused mixture-of-experts op of track 03 (include/fused_moe.h).
//
// Math (track-03/reference/reference.py:10-35), per token t: fp32 softmax of
// the bf16 router scores, the topk largest (lower expert index first on
// ties), optional renormalisation, bf16 weights; per selected expert e:
// x = bf16(h . w1[e]^T), u = bf16(x[N:] * bf16(silu(x[:N]))),
// y = bf16(u . w2[e]^T); out[t] = bf16 running sum over the selected experts
// in ascending order of bf16(y * w_e). Every bf16 rounding sits where the
// reference's bf16 tensors round, so the HIP path differs from the oracle
// only by the order of the fp32 sums inside the two GEMMs.
//
// Kernels of one call
// -------------------
// fm_route_kernel   one wave per token: softmax over E, top-k by repeated
//   wave-wide argmax on (weight, lower index), ids and bf16 weights written
//   in ascending expert order (the order of the final sum).
// fm_plan_kernel    one work-group: pairs (t, slot) counted per expert and
//   listed by expert, tiles of up to `tile_rows` pairs of one expert.
// fm_gemm_kernel<gated>   (tokens per expert > ~24) a tile of 128 pairs x
//   256 weight rows per work-group, K in 64-wide stages through a 3-stage
//   LDS ring filled by LDS-DMA (1 KiB per wave instruction, XOR-swizzled so
//   the MFMA fragment reads are free of bank conflicts), 32x32x16 bf16 MFMA,
//   fp32 accumulation. gated: w1 rows j (gate) and N + j (up) sit in the
//   same lane and register, so silu(gate) * up is formed in the epilogue.
//   Otherwise (w2): the epilogue multiplies by the pair's routing weight.
// fm_skinny_kernel<gated, PB>  (few tokens per expert: decode) the weights
//   are the streamed operand: each wave loads its 32 weight rows' MFMA
//   fragments straight from HBM into registers (8 k-steps, 24-32 KiB, in
//   flight per wave), the 16 * PB pairs' fragments likewise (L2-resident),
//   and the 4 waves of a work-group split K and add their partial sums
//   through LDS. 16x16x32 bf16 MFMA.
// fm_reduce_kernel  out[t] = bf16 running sum of the token's topk weighted
//   expert outputs, ascending expert order. Not launched when topk <= 2 and
//   the tiles are streamed (decode): the routing launch clears out, and the
//   down GEMM adds each weighted row into it with packed bf16 atomics (the
//   two-term bf16 sum does not depend on the order).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "fused_moe.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kMaxExperts = 256;
constexpr int kMaxTopk = 32;

// ---------------------------------------------------------------------------
// workspace plan (host)
// ---------------------------------------------------------------------------
constexpr int kLargeRows = 128;   // pairs per tile of fm_gemm_kernel
constexpr int kLargeCols = 256;   // weight rows per tile of fm_gemm_kernel
constexpr int kBK = 64;           // k per LDS stage
constexpr int kStages = 3;

struct Plan {
  int64_t P;            // pairs = M * topk
  int tile_rows;        // pairs per tile
  bool large;           // fm_gemm_kernel (else fm_skinny_kernel)
  bool big;             // large, with 256-pair tiles: fm_gemm_big_kernel
  int pb;               // small tiles: 16-pair blocks per tile (1, 2 or 4)
  int64_t max_tiles;    // upper bound on sum_e ceil(count_e / tile_rows)
  size_t ids_off, wts_off, eoff_off, sorted_off, tiles_off, inter_off, y_off, bytes;
};

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

Plan make_plan(const fm_args* a) {
  Plan p{};
  p.P = a->M * a->topk;
  const double avg = double(p.P) / double(a->E);  // pairs per expert on average
  if (a->flags & (FM_FLAG_LARGE_TILES | FM_FLAG_BIG_TILES))
    p.large = true;
  else if (a->flags & FM_FLAG_SMALL_TILES)
    p.large = false;
  else
    p.large = avg > 24.0;
  // 256-pair tiles when an expert's pairs fill them well and their gate-up
  // GEMM still has a work-group for each of MI355X's 256 CUs (P / 256 pair
  // tiles x N / 128 column tiles; fewer, and the 128-pair tiles' larger grid
  // is faster: measured at M = 1024, 2048 with E = 8). Which fills better
  // depends on the pairs per expert (K = 2048, N = 1024, E = 64, whole
  // calls): 256-pair tiles win at 136-192 on average (most experts fit one,
  // 4-8 %) and from 384 on; 128-pair tiles below 130 and at 225-336, where
  // many experts spill a few pairs into a second, nearly empty 256-pair tile
  // (2-10 %).
  const bool fills = (avg >= 128.0 && avg < 208.0) || avg >= 360.0;
  p.big = (a->flags & FM_FLAG_BIG_TILES) != 0 ||
          ((a->flags & FM_FLAG_LARGE_TILES) == 0 && p.large && fills &&
           (p.P / 256) * (a->N / 128) >= 256);
  // 16 or 32 pairs per small tile (64 only when forced; measured slower than
  // the large tiles at 48 pairs per expert)
  p.pb = avg > 24.0 && a->N % 256 == 0 ? 4 : avg > 12.0 ? 2 : 1;
  p.tile_rows = p.big ? 256 : p.large ? kLargeRows : 16 * p.pb;
  const int64_t nonempty = a->E < p.P ? a->E : p.P;
  p.max_tiles = p.P / p.tile_rows + nonempty;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = round_up(off + bytes, 256);
    return o;
  };
  p.ids_off = take(size_t(p.P) * 4);
  p.wts_off = take(size_t(p.P) * 4);
  p.eoff_off = take(size_t(a->E + 1) * 4);
  p.sorted_off = take(size_t(p.P) * 4);
  p.tiles_off = take(16 + size_t(p.max_tiles) * 16);  // count, then int4 per tile
  p.inter_off = take(size_t(p.P) * size_t(a->N) * 2);
  p.y_off = take(size_t(p.P) * size_t(a->K) * 2);
  p.bytes = off;
  return p;
}

int validate(const fm_args* a) {
  if (a == nullptr) return FM_EINVAL;
  if (a->M < 0 || a->K <= 0 || a->N <= 0 || a->E <= 0 || a->topk <= 0) return FM_EINVAL;
  if (a->topk > a->E) return FM_EINVAL;
  if (a->E > kMaxExperts || a->topk > kMaxTopk) return FM_EUNSUPPORTED;
  if (a->K % kLargeCols != 0 || a->N % (kLargeCols / 2) != 0) return FM_EUNSUPPORTED;
  const uint32_t tile_flags = a->flags & (FM_FLAG_LARGE_TILES | FM_FLAG_SMALL_TILES |
                                          FM_FLAG_BIG_TILES);
  if ((a->flags & ~(tile_flags | FM_FLAG_ORDERED_SUM)) != 0 ||
      (tile_flags & (tile_flags - 1)) != 0)
    return FM_EINVAL;  // unknown bits, or more than one tile choice
  if (a->M == 0) return FM_OK;
  if (!a->hidden || !a->w1 || !a->w2 || !a->score || !a->out) return FM_EINVAL;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!al16(a->hidden) || !al16(a->w1) || !al16(a->w2) || !al16(a->out)) return FM_EINVAL;
  if ((reinterpret_cast<uintptr_t>(a->score) & 1u) != 0) return FM_EINVAL;
  if (a->s_hidden < a->K || a->s_hidden % 8 != 0 || a->s_out < a->K || a->s_out % 8 != 0 ||
      a->s_score < a->E)
    return FM_EINVAL;
  // 32-bit byte offsets: rows of hidden, of one expert's weights and of the
  // intermediate buffers
  const int64_t lim = int64_t(UINT32_MAX) - 4096;
  if ((a->M - 1) * a->s_hidden * 2 + a->K * 2 > lim) return FM_EUNSUPPORTED;
  if (2 * a->N * a->K * 2 > lim) return FM_EUNSUPPORTED;
  if (a->M * a->topk * a->N * 2 > lim || a->M * a->topk * a->K * 2 > lim) return FM_EUNSUPPORTED;
  return FM_OK;
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16r(float x) {  // round to the nearest bf16
  return static_cast<float>(static_cast<__bf16>(x));
}

// silu in fp32, as torch's bf16 silu computes it before its rounding
__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long y = __shfl_xor(x, o);
    x = y > x ? y : x;
  }
  return x;
}

// LDS-DMA of 16 bytes per lane from SGPR base + 32-bit lane offset into
// LDS bytes lds_addr + 16 * lane. The LDS address is handed to the compiler
// as the M0 operand; s_nop 0 covers the wait state after its write. The
// compiler does not see the LDS write: the caller waits (vmcnt) and
// synchronizes before the data is read.
__device__ __forceinline__ void lds_dma(const void* base, uint32_t lane_off, uint32_t lds_addr) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(lane_off), "s"(base), "{m0}"(lds_addr)
      : "memory");
}

// Work-group barrier that orders LDS traffic only (lgkmcnt = 0, then
// s_barrier): LDS-DMA loads issued earlier keep flying across it, where
// __syncthreads() would drain every outstanding global load.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt = max, expcnt = max, lgkmcnt = 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) for a wave-uniform n known only at run time.
__device__ __forceinline__ void wait_vmcnt(int n) {  // n uniform, 0..24
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
    case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
    case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
  }
}

// ============================================================================
// routing
// ============================================================================
struct RouteParams {
  const __bf16* score;
  int64_t s_score;
  int32_t* ids;     // [M, topk] ascending expert ids
  float* wts;       // [M, topk] bf16-rounded weights (as fp32)
  int64_t M;
  int E, topk, renormalize;
  // when the down GEMM adds into the output itself: the rows to clear
  __bf16* zero_out;
  int64_t s_out;
  int K;
};

// Clears output row t (K bf16, 16-byte aligned) by one wave.
__device__ __forceinline__ void clear_out_row(const RouteParams& p, int64_t t, int lane) {
  __bf16* row = p.zero_out + t * p.s_out;
  bf16x8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = static_cast<__bf16>(0.f);
  for (int k = 8 * lane; k < p.K; k += 8 * 64) *reinterpret_cast<bf16x8*>(row + k) = z;
}

// Routing of token t by one wave; lane l holds experts l, l + 64, l + 128,
// l + 192. `raw` are the token's scores as loaded (bf16 widened; -inf past E).
constexpr int kPer = kMaxExperts / 64;
__device__ __forceinline__ void load_scores(const RouteParams& p, int64_t t, int lane,
                                            float (&raw)[kPer]) {
  const __bf16* srow = p.score + t * p.s_score;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e = lane + 64 * i;
    raw[i] = e < p.E ? static_cast<float>(srow[e]) : -INFINITY;
  }
}

__device__ __forceinline__ void route_token(const RouteParams& p, int64_t t, int lane,
                                            const float (&raw)[kPer]) {
  float v[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    v[i] = raw[i];
    mx = fmaxf(mx, v[i]);
  }
  mx = wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    v[i] = (lane + 64 * i) < p.E ? expf(v[i] - mx) : 0.f;
    sum += v[i];
  }
  sum = wave_sum(sum);
#pragma unroll
  for (int i = 0; i < kPer; ++i) v[i] = v[i] / sum;  // softmax weight (>= 0)
  // top-k: repeated argmax over (weight, lower index); a weight's bits order
  // like its value (weights are >= 0), the index goes in complemented
  bool sel[kPer] = {};
  float tot = 0.f;  // sum of the selected weights, in selection order
  for (int r = 0; r < p.topk; ++r) {
    unsigned long long key = 0ull;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = lane + 64 * i;
      if (e < p.E && !sel[i]) {
        const unsigned long long k = (static_cast<unsigned long long>(__float_as_uint(v[i])) << 32) |
                                     (0xFFFFFFFFu - unsigned(e));
        key = k > key ? k : key;
      }
    }
    key = wave_max_u64(key);
    const int win = int(0xFFFFFFFFu - unsigned(key & 0xFFFFFFFFull));
    tot += __uint_as_float(unsigned(key >> 32));
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (lane + 64 * i == win) sel[i] = true;
  }
  // ascending-expert slot of each selected expert: ballots in expert order
  int before = 0;
  const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const unsigned long long m = __ballot(sel[i]);
    if (sel[i]) {
      const int slot = before + __popcll(m & below);
      const float w = p.renormalize ? v[i] / tot : v[i];
      p.ids[t * p.topk + slot] = lane + 64 * i;
      p.wts[t * p.topk + slot] = bf16r(w);
    }
    before += __popcll(m);
  }
}

// One wave per token.
__global__ void __launch_bounds__(256) fm_route_kernel(const RouteParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= p.M) return;
  float raw[kPer];
  load_scores(p, t, lane, raw);
  route_token(p, t, lane, raw);
  if (p.zero_out != nullptr) clear_out_row(p, t, lane);
}

// ============================================================================
// plan: pairs by expert, tiles
// ============================================================================
struct PlanParams {
  const int32_t* ids;
  int32_t* eoff;      // [E + 1] first sorted position of each expert
  int32_t* sorted;    // [P] pair ids (t * topk + slot) grouped by expert
  int32_t* tiles;     // [0] = tile count, then int4 (expert, start, rows, 0) per tile
  int64_t P;
  int E, tile_rows;
};

struct PlanSmem {
  int cnt[kMaxExperts];
  int off[kMaxExperts + 1];
  int toff[kMaxExperts + 1];
  int cur[kMaxExperts];
};

// The plan, by the 1024 threads of one work-group.
__device__ __forceinline__ void plan_body(const PlanParams& p, PlanSmem& sm) {
  int* s_cnt = sm.cnt;
  int* s_off = sm.off;
  int* s_toff = sm.toff;
  int* s_cur = sm.cur;
  const int tid = threadIdx.x;
  for (int e = tid; e < kMaxExperts; e += 1024) {
    s_cnt[e] = 0;
    s_cur[e] = 0;
  }
  __syncthreads();
  for (int64_t i = tid; i < p.P; i += 1024) atomicAdd(&s_cnt[p.ids[i]], 1);
  __syncthreads();
  if (tid < 64) {  // exclusive scans of counts and tile counts over <= 256 experts
    int carry = 0, tcarry = 0;
    for (int c = 0; c < kMaxExperts / 64; ++c) {
      const int e = 64 * c + tid;
      const int v = e < p.E ? s_cnt[e] : 0;
      const int tv = (v + p.tile_rows - 1) / p.tile_rows;
      int incl = v, tincl = tv;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int a = __shfl_up(incl, o);
        const int b = __shfl_up(tincl, o);
        if (tid >= o) {
          incl += a;
          tincl += b;
        }
      }
      if (e < p.E) {
        s_off[e] = carry + incl - v;
        s_toff[e] = tcarry + tincl - tv;
      }
      carry += __shfl(incl, 63);
      tcarry += __shfl(tincl, 63);
    }
    if (tid == 0) {
      s_off[p.E] = carry;
      s_toff[p.E] = tcarry;
    }
  }
  __syncthreads();
  for (int e = tid; e <= p.E; e += 1024) p.eoff[e] = s_off[e];
  if (tid == 0) p.tiles[0] = s_toff[p.E];
  for (int64_t i = tid; i < p.P; i += 1024) {
    const int e = p.ids[i];
    p.sorted[s_off[e] + atomicAdd(&s_cur[e], 1)] = int32_t(i);
  }
  for (int e = tid; e < p.E; e += 1024) {
    const int n = s_cnt[e];
    for (int k = 0; k * p.tile_rows < n; ++k) {
      int32_t* tl = p.tiles + 4 + 4 * (s_toff[e] + k);
      tl[0] = e;
      tl[1] = s_off[e] + k * p.tile_rows;
      tl[2] = min(p.tile_rows, n - k * p.tile_rows);
      tl[3] = 0;
    }
  }
}

__global__ void __launch_bounds__(1024) fm_plan_kernel(const PlanParams p) {
  __shared__ PlanSmem sm;
  plan_body(p, sm);
}

// Few tokens (decode): routing and plan in one work-group, one launch fewer.
// Wave w routes token w. (With 4 tokens per wave, at M = 64, the one
// work-group took 18.5 us against 6.5 + 6.5 for the two launches.)
constexpr int kFusedRouteTokens = 16;
__global__ void __launch_bounds__(1024) fm_route_plan_kernel(const RouteParams rp,
                                                             const PlanParams pp) {
  __shared__ PlanSmem sm;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  constexpr int kPerWave = kFusedRouteTokens / 16;
  float raw[kPerWave][kPer];
#pragma unroll
  for (int j = 0; j < kPerWave; ++j) {
    const int64_t t = wave + 16 * j;
    if (t < rp.M) load_scores(rp, t, lane, raw[j]);
  }
#pragma unroll
  for (int j = 0; j < kPerWave; ++j) {
    const int64_t t = wave + 16 * j;
    if (t < rp.M) {
      route_token(rp, t, lane, raw[j]);
      if (rp.zero_out != nullptr) clear_out_row(rp, t, lane);
    }
  }
  // the ids and weights are in memory before any thread of the group reads
  // them back (same CU: the workgroup barrier orders them once stored)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  plan_body(pp, sm);
}

// ============================================================================
// GEMMs
// ============================================================================
// GEMM 1 (gated): A row r of a tile = hidden[token of pair sorted[start + r]],
//   weight rows = w1[e] rows j (gate) and N + j (up); output u to
//   inter[start + r, j] (sorted pair order).
// GEMM 2: A row r = inter[start + r], weight rows = w2[e] rows f (features);
//   output bf16(bf16(y) * w_pair) to yw[pair, f] (pair = t * topk + slot).
struct GemmParams {
  const __bf16* a;       // hidden or inter
  int64_t a_stride;      // elements per A row
  const __bf16* w;       // w1 or w2
  int64_t w_estride;     // elements per expert
  const int32_t* sorted;
  const int32_t* tiles;  // [0] = count, then int4 per tile
  const float* wts;      // routing weights by pair (GEMM 2)
  __bf16* out;           // inter [P, N] or yw [P, K]
  int64_t out_stride;    // elements per output row
  int kin;               // reduction length: K (GEMM 1) or N (GEMM 2)
  int nout;              // GEMM 1: N (gate rows; up rows follow); GEMM 2: K
  int topk;
  int col_tiles;         // output-column tiles per pair tile
  int ct_per_wg;         // column tiles one work-group runs (fm_stream_kernel)
  int xcd_grid;          // large/big tiles: the 2 x 4 XCD grid of xcd_item
  // GEMM 2 with topk <= 2 (fm_stream_kernel): add each pair's bf16 row into
  // the token's output row instead of writing yw (null: write yw)
  __bf16* fsum;
  int64_t fsum_stride;
};

// out[0..1] += (a0, a1) as one packed bf16 atomic add at agent scope (sc1:
// performed where every XCD sees it; the two addends of an element may come
// from work-groups on different XCDs). Each element gets at most two addends
// onto the cleared 0, so the result is bf16(x + y): the reference's ascending
// running sum, whose two-term form does not depend on the order.
__device__ __forceinline__ void add_bf16x2(__bf16* out, __bf16 a0, __bf16 a1) {
  const uint32_t v = uint32_t(__builtin_bit_cast(uint16_t, a0)) |
                     uint32_t(__builtin_bit_cast(uint16_t, a1)) << 16;
  asm volatile("global_atomic_pk_add_bf16 %0, %1, off sc1" : : "v"(out), "v"(v) : "memory");
}

// Work item (pair tile, column tile) of a large or big GEMM work-group.
// Work-group b runs on XCD b % 8 (dispatch is round-robin over the XCDs, in
// order of b). Plainly, b -> (b / col_tiles, b % col_tiles): column tile c of
// every pair tile runs on XCD c % 8, so a weight tile is read into one L2 and
// shared there by the pair tiles of its expert, while every pair tile's
// gathered A rows are read into col_tiles L2s. With p.xcd_grid the XCDs form
// a 2 x 4 grid instead: XCD x takes the column tiles of half x % 2 of every
// pair tile in its contiguous quarter x / 2 of the tile table, pair tile by
// pair tile, so a pair tile's A rows go to two L2s, and an expert's pair
// tiles (adjacent in the table) still share its weight rows in one L2.
// The host sets xcd_grid when experts average fewer than two pair tiles and
// the items outnumber the CUs. Measured at K = 2048, N = 1024 (gate-up +
// down): M = 4096, E = 64, topk = 6 (1.5 pair tiles per expert) 5-10 %
// faster; M = 512-3072 at E = 64, 1-7 %; but M = 4096, E = 8, topk = 2 (4
// pair tiles per expert) 20 % slower with one set of routings and level with
// another, and M = 8192, E = 8 8 % slower. Whole column tiles on each XCD
// (an 8 x 1 grid) gained 10 % at M = 4096, E = 64 and lost 15 % at E = 8.
// False: no item for this work-group.
constexpr int kXcds = 8;
constexpr int kXcdColGroups = 2;
constexpr int kXcdTileGroups = kXcds / kXcdColGroups;

__device__ __forceinline__ bool xcd_item(const GemmParams& p, int& tile, int& ct) {
  const int nt = p.tiles[0];
  const int b = int(blockIdx.x);
  if (!p.xcd_grid) {
    tile = b / p.col_tiles;
    ct = b % p.col_tiles;
    return tile < nt;
  }
  const int x = b % kXcds, s = b / kXcds;
  const int cg = x % kXcdColGroups, tg = x / kXcdColGroups;
  const int c0 = cg * p.col_tiles / kXcdColGroups;
  const int cn = (cg + 1) * p.col_tiles / kXcdColGroups - c0;
  const int t0 = tg * nt / kXcdTileGroups;
  const int tn = (tg + 1) * nt / kXcdTileGroups - t0;
  if (cn <= 0 || s >= tn * cn) return false;
  tile = t0 + s / cn;
  ct = c0 + s % cn;
  return true;
}

// ---- large tiles -------------------------------------------------------------
// LDS stage: A 128 rows x 128 B, then B 256 rows x 128 B. Row r's 16-byte
// chunk c (k = 8c..8c+7 of the stage) sits at chunk position c ^ ((r >> 1) & 7):
// a 32x32x16 fragment read (lanes 0..15 = 16 consecutive rows, one chunk)
// then covers all 64 banks once. An LDS-DMA instruction writes 8 rows
// (1 KiB) lane-linearly, so each lane loads the global chunk that belongs at
// its position.
constexpr int kRowBytes = kBK * 2;                  // 128
constexpr int kAStage = kLargeRows * kRowBytes;     // 16 KiB
constexpr int kBStage = kLargeCols * kRowBytes;     // 32 KiB
constexpr int kStage = kAStage + kBStage;           // 48 KiB

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// The K loop and epilogue of one tile with NRB row blocks (of 32 pairs)
// holding pairs: full tiles run NRB = 4, an expert's last tile fewer.
template <bool kGated, int NRB>
__device__ __forceinline__ void gemm_tile(const GemmParams& p, uint8_t* s_buf, const int* s_pair,
                                          const float* s_wt, const uint8_t* abase,
                                          const uint8_t* wbase, const uint32_t (&a_off)[4],
                                          const uint32_t (&b_off)[8], uint32_t lds0, int start,
                                          int rows, int ct) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int nst = p.kin / kBK;
  // A instructions of this wave that hold a pair (rows 32 * wave + 8 * g ..):
  // the rows past the tile's last pair are never loaded (nor read)
  const int na = max(0, min(4, (rows - 32 * wave + 7) / 8));
  // DMA d (0..11) of a stage: A instruction d (d < 4), else B instruction d - 4
  auto dma = [&](int st, int d) {
    const uint32_t sb = lds0 + uint32_t((st % kStages) * kStage);
    if (d < 4) {
      if (d < na)
        lds_dma(abase + int64_t(st) * kRowBytes, a_off[d], sb + uint32_t((4 * wave + d) * 1024));
    } else {
      lds_dma(wbase + int64_t(st) * kRowBytes, b_off[d - 4],
              sb + uint32_t(kAStage + (8 * wave + d - 4) * 1024));
    }
  };
  auto issue = [&](int st) {
#pragma unroll
    for (int d = 0; d < 12; ++d) dma(st, d);
  };

  f32x16 acc[NRB][2];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][cb][i] = 0.f;

  issue(0);
  if (nst > 1) issue(1);
  for (int st = 0; st < nst; ++st) {
    // this wave's loads of stage st are complete (na + 8 per stage; the
    // ones of stage st + 1 may still fly), then every wave's are
    wait_vmcnt(st + 1 < nst ? na + 8 : 0);
    lds_barrier();
    // stage st + 2 goes into the buffer every wave finished reading; its 12
    // DMAs are spread over this stage's MFMAs (one per 2 MFMAs at NRB = 4)
    const bool more = st + 2 < nst;
    const uint8_t* sa = s_buf + (st % kStages) * kStage;
    const uint8_t* sb = sa + kAStage;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int c = 2 * kk + hi;
      bf16x8 bf[2];
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int lr = 64 * wave + 32 * cb + l32;
        bf[cb] = *reinterpret_cast<const bf16x8*>(sb + lr * kRowBytes + swz(lr, c) * 16);
      }
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        const int r = 32 * rb + l32;
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(sa + r * kRowBytes + swz(r, c) * 16);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf[cb], acc[rb][cb], 0, 0, 0);
        constexpr int kSlots = 4 * NRB;  // MFMA pairs per stage
        const int slot = kk * NRB + rb;
        if (more) {
#pragma unroll
          for (int d = (slot * 12) / kSlots; d < ((slot + 1) * 12) / kSlots; ++d) dma(st + 2, d);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the DMAs between the MFMAs
      }
    }
  }

  // epilogue: lane holds column l32 of each column block and pair rows
  // 32 * rb + 8 * a + 4 * hi + b in register 4 * a + b
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int r = 32 * rb + 8 * a + 4 * hi + b;
        if (r >= rows) continue;
        const int ri = 4 * a + b;
        if (kGated) {
          const float g = bf16r(silu(bf16r(acc[rb][0][ri])));
          const float u = bf16r(acc[rb][1][ri]) * g;
          const int j = ct * (kLargeCols / 2) + 32 * wave + l32;
          p.out[int64_t(start + r) * p.out_stride + j] = static_cast<__bf16>(u);
        } else {
          const int pair = s_pair[r];
          const float w = s_wt[r];
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) {
            const int f = ct * kLargeCols + 64 * wave + 32 * cb + l32;
            p.out[int64_t(pair) * p.out_stride + f] =
                static_cast<__bf16>(bf16r(acc[rb][cb][ri]) * w);
          }
        }
      }
  }
}

template <bool kGated>
__global__ void __launch_bounds__(256, 1) fm_gemm_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t s_buf[kStages * kStage];
  __shared__ int s_pair[kLargeRows];
  __shared__ float s_wt[kLargeRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tile, ct;
  if (!xcd_item(p, tile, ct)) return;
  const int32_t* tl = p.tiles + 4 + 4 * tile;
  const int e = __builtin_amdgcn_readfirstlane(tl[0]);
  const int start = __builtin_amdgcn_readfirstlane(tl[1]);
  const int rows = __builtin_amdgcn_readfirstlane(tl[2]);

  if (tid < kLargeRows) {
    const int r = tid < rows ? tid : 0;
    const int pair = p.sorted[start + r];
    s_pair[tid] = pair;
    if (!kGated) s_wt[tid] = p.wts[pair];
  }
  __syncthreads();

  // Per-lane DMA sources. A: this wave's 4 instructions cover tile rows
  // 32 * wave + 8 * g + lane / 8; B: its 8 instructions cover its own 64
  // weight rows (LDS rows 64 * wave + 8 * g + lane / 8).
  const int sub = lane >> 3;       // row within the instruction's 8
  const int pos = lane & 7;        // chunk position within the row
  uint32_t a_off[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int r = 32 * wave + 8 * g + sub;
    const int c = swz(r, pos);  // the chunk whose swizzled position is `pos`
    const int64_t arow = kGated ? int64_t(s_pair[r] / p.topk) : int64_t(start + (r < rows ? r : 0));
    a_off[g] = uint32_t(arow * p.a_stride * 2 + c * 16);
  }
  uint32_t b_off[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const int lr = 64 * wave + 8 * g + sub;   // LDS row of the B stage
    const int cb = (lr >> 5) & 1;             // column block of the wave
    const int i = lr & 31;
    int wrow;
    if (kGated)  // gate rows j, up rows N + j, j = ct * 128 + 32 * wave + i
      wrow = (cb ? p.nout : 0) + ct * (kLargeCols / 2) + 32 * wave + i;
    else         // features f = ct * 256 + lr
      wrow = ct * kLargeCols + lr;
    b_off[g] = uint32_t(int64_t(wrow) * p.kin * 2 + swz(lr, pos) * 16);
  }
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(p.a);
  const uint8_t* wbase = reinterpret_cast<const uint8_t*>(p.w + int64_t(e) * p.w_estride);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      uint32_t(reinterpret_cast<uintptr_t>((lds_u8_t*)s_buf)));

  const int nrb = (rows + 31) / 32;  // 32-pair row blocks holding pairs
#define FM_TILE(n) \
  gemm_tile<kGated, n>(p, s_buf, s_pair, s_wt, abase, wbase, a_off, b_off, lds0, start, rows, ct)
  switch (nrb) {
    case 1: FM_TILE(1); break;
    case 2: FM_TILE(2); break;
    case 3: FM_TILE(3); break;
    default: FM_TILE(4); break;
  }
#undef FM_TILE
}

// ---- big tiles (many pairs per expert) -----------------------------------------------
// Work-group: 256 pairs x 256 weight rows, 8 waves, two per SIMD. Wave w
// computes pair half w >> 2 (128 pairs, 4 row blocks) against weight quarter
// w & 3 (64 rows, 2 column blocks): the 128-pair tile's per-wave shape, with
// each weight fragment now feeding 256 pairs and each pair fragment 256 rows,
// so a stage moves 128 flop per byte into LDS (85 for the 128-pair tile), and
// the second wave on each SIMD issues MFMAs while the first waits for its
// fragment reads. K streams in 32-wide stages through a 4-deep ring (32 KiB
// per stage: A 256 rows, then B 256 rows, of 64 bytes), in pairs: two stages
// are in flight while the other two are read. Row r's 16-byte chunk c sits at
// c ^ ((r >> 2) & 3):
// 16 consecutive rows of one chunk (a fragment read's LDS cycle) then hit 16
// distinct groups of 4 banks. Each wave moves A rows 32w..32w+31 and B rows
// 32w..32w+31 of every stage (two 16-row LDS-DMA instructions each; A rows
// past the tile's last pair are skipped).
constexpr int kBigRows = 256;                        // pairs per tile
constexpr int kBigBK = 32;                           // k per stage
constexpr int kBigStages = 4;
constexpr int kBigRowBytes = kBigBK * 2;             // 64
constexpr int kBigAStage = kBigRows * kBigRowBytes;  // 16 KiB
constexpr int kBigStage = 2 * kBigAStage;            // A then B (256 weight rows)
static_assert(kLargeCols == 256, "the big tile's weight rows are the large tile's");

__device__ __forceinline__ int swz4(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

// The K loop and epilogue of one wave's share of a big tile; NRB = the 32-pair
// row blocks of the wave's half holding pairs (0: DMAs and barriers only).
template <bool kGated, int NRB>
__device__ __forceinline__ void big_tile(const GemmParams& p, const uint8_t* s_buf,
                                         const int* s_pair, const float* s_wt,
                                         const uint8_t* abase, const uint8_t* wbase,
                                         const uint32_t (&a_off)[2], const uint32_t (&b_off)[2],
                                         uint32_t lds0, int na, int start, int rows, int ct) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ph = wave >> 2;  // pair half
  const int wq = wave & 3;   // weight quarter
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int nst = p.kin / kBigBK;
  auto issue = [&](int st) {
    const uint32_t sb = lds0 + uint32_t((st % kBigStages) * kBigStage);
    const int64_t k0 = int64_t(st) * kBigRowBytes;
#pragma unroll
    for (int g = 0; g < 2; ++g)
      if (g < na) lds_dma(abase + k0, a_off[g], sb + uint32_t((2 * wave + g) * 1024));
#pragma unroll
    for (int g = 0; g < 2; ++g)
      lds_dma(wbase + k0, b_off[g], sb + uint32_t(kBigAStage + (2 * wave + g) * 1024));
  };

  f32x16 acc[NRB > 0 ? NRB : 1][2];
#pragma unroll
  for (int rb = 0; rb < (NRB > 0 ? NRB : 1); ++rb)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][cb][i] = 0.f;

  // Stages go in pairs: one wait and barrier per pair. Before pair (st,
  // st + 1) only its own loads are in flight; after the barrier the next
  // pair's are issued into the buffers of the pair every wave has just
  // finished (one barrier per 64 k instead of per 32: 1-7 % faster).
  static_assert(kBigStages == 4, "two pairs of stage buffers");
  for (int st = 0; st < 2 && st < nst; ++st) issue(st);
  // one stage's fragment reads (both k-steps) and MFMAs
  auto reads = [&](int st, bf16x8 (&bf)[2][2], bf16x8 (&af)[2][NRB > 0 ? NRB : 1]) {
    const uint8_t* sa = s_buf + (st % kBigStages) * kBigStage;
    const uint8_t* sb = sa + kBigAStage;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = 2 * kk + hi;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int lr = 64 * wq + 32 * cb + l32;
        bf[kk][cb] = *reinterpret_cast<const bf16x8*>(sb + lr * kBigRowBytes + swz4(lr, c) * 16);
      }
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        const int r = 128 * ph + 32 * rb + l32;
        af[kk][rb] = *reinterpret_cast<const bf16x8*>(sa + r * kBigRowBytes + swz4(r, c) * 16);
      }
    }
  };
  auto mfmas = [&](const bf16x8 (&bf)[2][2], const bf16x8 (&af)[2][NRB > 0 ? NRB : 1]) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk][rb], bf[kk][cb],
                                                                 acc[rb][cb], 0, 0, 0);
  };
  // nst is even: validate() requires K % 256 == 0 and N % 128 == 0
  for (int st = 0; st < nst; st += 2) {
    wait_vmcnt(0);
    lds_barrier();
    for (int s2 = st + 2; s2 < st + 4 && s2 < nst; ++s2) issue(s2);
    if constexpr (NRB > 0) {
      // the pair in one body: the second stage's fragment reads fly under
      // the first's MFMAs (1-4 % against a loop over single stages)
      bf16x8 bf0[2][2], af0[2][NRB], bf1[2][2], af1[2][NRB];
      reads(st, bf0, af0);
      reads(st + 1, bf1, af1);
      mfmas(bf0, af0);
      mfmas(bf1, af1);
    }
  }

  // epilogue: lane holds column l32 of each column block and pair rows
  // 128 * ph + 32 * rb + 8 * a + 4 * hi + b in register 4 * a + b
  if constexpr (NRB > 0) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int r = 128 * ph + 32 * rb + 8 * a + 4 * hi + b;
          if (r >= rows) continue;
          const int ri = 4 * a + b;
          if (kGated) {
            const float g = bf16r(silu(bf16r(acc[rb][0][ri])));
            const float u = bf16r(acc[rb][1][ri]) * g;
            const int j = ct * (kLargeCols / 2) + 32 * wq + l32;
            p.out[int64_t(start + r) * p.out_stride + j] = static_cast<__bf16>(u);
          } else {
            const int pair = s_pair[r];
            const float w = s_wt[r];
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
              const int f = ct * kLargeCols + 64 * wq + 32 * cb + l32;
              p.out[int64_t(pair) * p.out_stride + f] =
                  static_cast<__bf16>(bf16r(acc[rb][cb][ri]) * w);
            }
          }
        }
    }
  }
}

template <bool kGated>
__global__ void __launch_bounds__(512, 1) fm_gemm_big_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t s_buf[kBigStages * kBigStage];
  __shared__ int s_pair[kBigRows];
  __shared__ float s_wt[kBigRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  int tile, ct;
  if (!xcd_item(p, tile, ct)) return;
  const int32_t* tl = p.tiles + 4 + 4 * tile;
  const int e = __builtin_amdgcn_readfirstlane(tl[0]);
  const int start = __builtin_amdgcn_readfirstlane(tl[1]);
  const int rows = __builtin_amdgcn_readfirstlane(tl[2]);

  if (tid < kBigRows) {
    const int r = tid < rows ? tid : 0;
    const int pair = p.sorted[start + r];
    s_pair[tid] = pair;
    if (!kGated) s_wt[tid] = p.wts[pair];
  }
  __syncthreads();

  // Per-lane DMA sources: instruction g of this wave moves LDS rows
  // 32 * wave + 16 * g + lane / 4, lane & 3 being the chunk position there.
  const int sub = lane >> 2;
  const int pos = lane & 3;
  uint32_t a_off[2], b_off[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int r = 32 * wave + 16 * g + sub;
    const int c = swz4(r, pos);  // the chunk whose swizzled position is `pos`
    const int64_t arow =
        kGated ? int64_t(s_pair[r] / p.topk) : int64_t(start + (r < rows ? r : 0));
    a_off[g] = uint32_t(arow * p.a_stride * 2 + c * 16);
    // weight row of LDS row r: weight quarter r >> 6, column block (r >> 5) & 1
    int wrow;
    if (kGated)  // gate rows j, up rows N + j, j = ct * 128 + 32 * (r >> 6) + (r & 31)
      wrow = (((r >> 5) & 1) ? p.nout : 0) + ct * (kLargeCols / 2) + 32 * (r >> 6) + (r & 31);
    else         // features f = ct * 256 + r
      wrow = ct * kLargeCols + r;
    b_off[g] = uint32_t(int64_t(wrow) * p.kin * 2 + c * 16);
  }
  // A instructions of this wave that hold a pair
  const int na = max(0, min(2, (rows - 32 * wave + 15) / 16));
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(p.a);
  const uint8_t* wbase = reinterpret_cast<const uint8_t*>(p.w + int64_t(e) * p.w_estride);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      uint32_t(reinterpret_cast<uintptr_t>((lds_u8_t*)s_buf)));

  // 32-pair row blocks of this wave's half that hold pairs
  const int nrb = max(0, min(4, (rows - 128 * (wave >> 2) + 31) / 32));
#define FM_BIG(n)                                                                          \
  big_tile<kGated, n>(p, s_buf, s_pair, s_wt, abase, wbase, a_off, b_off, lds0, na, start, \
                      rows, ct)
  switch (nrb) {
    case 0: FM_BIG(0); break;
    case 1: FM_BIG(1); break;
    case 2: FM_BIG(2); break;
    case 3: FM_BIG(3); break;
    default: FM_BIG(4); break;
  }
#undef FM_BIG
}

// ---- skinny tiles (few pairs per expert) ------------------------------------------
// Work-group: one tile of up to 16 * PB pairs x 16 output rows (gated: 16
// gate rows j and the 16 up rows N + j; else 32 features in two blocks).
// Wave w takes k-steps w, w + 4, ... (32 k each): 16x16x32 MFMA with the
// weight rows as A (lane: row l % 16, k 8 * (l / 16)..+7 of the step) and the
// pairs as B, both loaded straight into registers, 8 k-steps per batch.
// D[weight row][pair]: lane holds pair l % 16, rows 4 * (l / 16) + i.
constexpr int kSkBatch = 8;

template <bool kGated, int PB>
__global__ void __launch_bounds__(256) fm_skinny_kernel(const GemmParams p) {
  __shared__ f32x4 s_red[4][2][PB][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;
  const int lg = lane >> 4;

  const int tile = int(blockIdx.x) / p.col_tiles;
  const int ct = int(blockIdx.x) % p.col_tiles;
  if (tile >= p.tiles[0]) return;
  const int32_t* tl = p.tiles + 4 + 4 * tile;
  const int e = tl[0];
  const int start = tl[1];
  const int rows = tl[2];

  // weight rows of this lane's A fragments (block 0 and 1)
  const __bf16* w = p.w + int64_t(e) * p.w_estride;
  const __bf16* wr[2];
  if (kGated) {
    wr[0] = w + int64_t(16 * ct + li) * p.kin;              // gate j
    wr[1] = w + int64_t(p.nout + 16 * ct + li) * p.kin;     // up j
  } else {
    wr[0] = w + int64_t(32 * ct + li) * p.kin;
    wr[1] = w + int64_t(32 * ct + 16 + li) * p.kin;
  }
  // pair rows of this lane's B fragments
  const __bf16* ar[PB];
#pragma unroll
  for (int q = 0; q < PB; ++q) {
    const int r = 16 * q + li;
    const int rr = r < rows ? r : 0;
    const int64_t arow = kGated ? int64_t(p.sorted[start + rr] / p.topk) : int64_t(start + rr);
    ar[q] = p.a + arow * p.a_stride;
  }

  f32x4 acc[2][PB];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int q = 0; q < PB; ++q) acc[b][q] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = p.kin / 32;
  for (int s0 = wave; s0 < nsteps; s0 += 4 * kSkBatch) {
    bf16x8 wf[kSkBatch][2];
    bf16x8 af[kSkBatch][PB];
#pragma unroll
    for (int u = 0; u < kSkBatch; ++u) {
      const int s = s0 + 4 * u;
      if (s < nsteps) {
        const int k = 32 * s + 8 * lg;
#pragma unroll
        for (int b = 0; b < 2; ++b) wf[u][b] = *reinterpret_cast<const bf16x8*>(wr[b] + k);
#pragma unroll
        for (int q = 0; q < PB; ++q) af[u][q] = *reinterpret_cast<const bf16x8*>(ar[q] + k);
      }
    }
#pragma unroll
    for (int u = 0; u < kSkBatch; ++u) {
      if (s0 + 4 * u < nsteps) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int q = 0; q < PB; ++q)
            acc[b][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[u][b], af[u][q], acc[b][q], 0,
                                                                 0, 0);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int q = 0; q < PB; ++q) s_red[wave][b][q][lane] = acc[b][q];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      f32x4 s = s_red[0][b][q][lane];
#pragma unroll
      for (int v = 1; v < 4; ++v) s += s_red[v][b][q][lane];  // fixed order: deterministic
      acc[b][q] = s;
    }
  // epilogue: pair r = 16 q + li, output rows 4 * lg + i
#pragma unroll
  for (int q = 0; q < PB; ++q) {
    const int r = 16 * q + li;
    if (r >= rows) continue;
    if (kGated) {
      bf16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float g = bf16r(silu(bf16r(acc[0][q][i])));
        o[i] = static_cast<__bf16>(bf16r(acc[1][q][i]) * g);
      }
      *reinterpret_cast<bf16x4*>(p.out + int64_t(start + r) * p.out_stride + 16 * ct + 4 * lg) = o;
    } else {
      const int pair = p.sorted[start + r];
      const float wt = p.wts[pair];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        bf16x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = static_cast<__bf16>(bf16r(acc[b][q][i]) * wt);
        *reinterpret_cast<bf16x4*>(p.out + int64_t(pair) * p.out_stride + 32 * ct + 16 * b +
                                   4 * lg) = o;
      }
    }
  }
}

// ---- streamed-weight tiles (decode) -------------------------------------------------
// Same work-group tile as fm_skinny_kernel (16 * PB pairs x 32 weight rows),
// but every operand reaches the MFMAs through LDS, filled by LDS-DMA in
// stages of 256 k: one instruction moves two rows' 512 contiguous bytes, so
// each weight row streams from HBM in long runs. Stages go through a ring of
// 3-6 buffers (all but one in flight); all waits are explicit (no
// compiler-tracked load shares the vmcnt counter with the DMAs). Pair rows
// past the tile's last pair are not loaded. Row r's 16-byte chunk c sits
// at position c ^ (r & 15) of its 512-byte line, so the 16 rows of a 16x16x32
// fragment read hit 16 distinct bank groups. The 4 waves split each stage's
// 8 k-steps (2 each) and add their partial sums through LDS at the end.
constexpr int kStK = 256;                 // k per stage
constexpr int kStLine = kStK * 2;         // 512 bytes per row per stage

template <bool kGated, int PB>
__global__ void __launch_bounds__(256, 1) fm_stream_kernel(const GemmParams p) {
  constexpr int kRowsW = 32;                        // weight rows per column tile
  constexpr int kRowsP = 16 * PB;                   // pair rows
  constexpr int kBuf = (kRowsW + kRowsP) * kStLine; // one stage
  constexpr int kDmaW = kRowsW / 2 / 4;             // weight DMAs per wave per stage (4)
  constexpr int kDmaP = kRowsP / 2 / 4;             // pair DMAs per wave per stage (2 PB)
  // ring depth: as many stages as 144 KiB of LDS hold (6, 4, 3)
  constexpr int kStBufs = (144 * 1024) / kBuf;
  static_assert(kStBufs >= 3 && 4 * 2 * PB * 64 * 16 <= kBuf, "ring and reduction fit");
  __shared__ __attribute__((aligned(1024))) uint8_t s_buf[kStBufs * kBuf];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15;
  const int lg = lane >> 4;

  // work-group: column tiles ct0 .. ct0 + p.ct_per_wg - 1 of one pair tile,
  // in one continuous stage pipeline
  const int wgs_per_tile = (p.col_tiles + p.ct_per_wg - 1) / p.ct_per_wg;
  const int tile = int(blockIdx.x) / wgs_per_tile;
  const int ct0 = (int(blockIdx.x) % wgs_per_tile) * p.ct_per_wg;
  if (tile >= p.tiles[0]) return;
  const int nct = min(p.ct_per_wg, p.col_tiles - ct0);
  const int32_t* tl = p.tiles + 4 + 4 * tile;
  const int e = __builtin_amdgcn_readfirstlane(tl[0]);
  const int start = __builtin_amdgcn_readfirstlane(tl[1]);
  const int rows = __builtin_amdgcn_readfirstlane(tl[2]);

  // DMA instruction g of a stage moves rows 2g, 2g + 1 (lane / 32 picks the
  // row, lane % 32 its chunk position); this wave issues weight instructions
  // kDmaW * wave + i and pair instructions kDmaP * wave + i. Offsets are for
  // column tile ct0; a later column tile moves the weight base.
  const int half = lane >> 5;
  const int posn = lane & 31;
  uint32_t w_off[kDmaW];
#pragma unroll
  for (int i = 0; i < kDmaW; ++i) {
    const int r = 2 * (kDmaW * wave + i) + half;  // weight row of the column tile, 0..31
    int wrow;
    if (kGated)  // rows 0..15: gate j = 16 ct + r; rows 16..31: up N + 16 ct + r - 16
      wrow = (r < 16 ? 0 : p.nout - 16) + 16 * ct0 + r;
    else
      wrow = 32 * ct0 + r;
    w_off[i] = uint32_t(int64_t(wrow) * p.kin * 2 + ((posn ^ (r & 15)) * 16));
  }
  uint32_t p_off[kDmaP];
#pragma unroll
  for (int i = 0; i < kDmaP; ++i) {
    const int r = 2 * (kDmaP * wave + i) + half;  // pair row of the tile, 0..16 PB - 1
    const int rr = r < rows ? r : 0;
    const int64_t arow = kGated ? int64_t(p.sorted[start + rr] / p.topk) : int64_t(start + rr);
    p_off[i] = uint32_t(arow * p.a_stride * 2 + ((posn ^ (r & 15)) * 16));
  }
  // pair instructions of this wave that hold a pair (rows 2 (kDmaP wave + i) ..)
  const int npd = max(0, min(kDmaP, (rows + 1) / 2 - kDmaP * wave));
  const int ndma = kDmaW + npd;  // DMAs of this wave per stage
  const uint8_t* wbase = reinterpret_cast<const uint8_t*>(p.w + int64_t(e) * p.w_estride);
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(p.a);
  // bytes between the weight rows of consecutive column tiles
  const int64_t ct_step = int64_t(kGated ? 16 : 32) * p.kin * 2;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(
      uint32_t(reinterpret_cast<uintptr_t>((lds_u8_t*)s_buf)));
  const int nst = p.kin / kStK;   // stages per column tile
  const int total = nct * nst;    // stages of the work-group
  auto issue = [&](int fs) {      // flat stage fs = column tile * nst + stage
    const int c = fs / nst, st = fs - c * nst;
    const uint32_t b = lds0 + uint32_t((fs % kStBufs) * kBuf);
    const uint8_t* wb = wbase + int64_t(c) * ct_step + int64_t(st) * kStLine;
    const uint8_t* ab = abase + int64_t(st) * kStLine;
#pragma unroll
    for (int i = 0; i < kDmaW; ++i)
      lds_dma(wb, w_off[i], b + uint32_t((kDmaW * wave + i) * 2 * kStLine));
#pragma unroll
    for (int i = 0; i < kDmaP; ++i)
      if (i < npd)
        lds_dma(ab, p_off[i], b + uint32_t(kRowsW * kStLine + (kDmaP * wave + i) * 2 * kStLine));
  };

  f32x4 acc[2][PB];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int q = 0; q < PB; ++q) acc[b][q] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int fs = 0; fs < total && fs < kStBufs - 1; ++fs) issue(fs);
  for (int fs = 0; fs < total; ++fs) {
    // this wave's DMAs of stage fs are complete (those of up to two later
    // stages may fly), then every wave's are
    wait_vmcnt(ndma * min(kStBufs - 2, total - 1 - fs));
    lds_barrier();
    if (fs + kStBufs - 1 < total) issue(fs + kStBufs - 1);  // into the buffer of stage fs - 1
    const uint8_t* bw = s_buf + (fs % kStBufs) * kBuf;
    const uint8_t* bp = bw + kRowsW * kStLine;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = (2 * wave + u) * 4 + lg;  // 16-byte chunk of this lane's k within the line
      bf16x8 wf[2], pf[PB];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int r = 16 * b + li;
        wf[b] = *reinterpret_cast<const bf16x8*>(bw + r * kStLine + ((c ^ (r & 15)) * 16));
      }
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        const int r = 16 * q + li;
        pf[q] = *reinterpret_cast<const bf16x8*>(bp + r * kStLine + ((c ^ (r & 15)) * 16));
      }
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int q = 0; q < PB; ++q)
          acc[b][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[b], pf[q], acc[b][q], 0, 0, 0);
    }
    if (fs % nst != nst - 1) continue;
    // ---- last stage of a column tile: add the waves' partial sums (fixed
    // order: deterministic); wave b < 2 finishes output block b
    const int ct = ct0 + fs / nst;
    // the partial sums go through this stage's buffer: every wave is done
    // with its operands (the barrier below), and the next DMA into it is
    // issued only after the next stage's barrier
    lds_barrier();
    f32x4(*s_red)[2][PB][64] = reinterpret_cast<f32x4(*)[2][PB][64]>(s_buf + (fs % kStBufs) * kBuf);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        s_red[wave][b][q][lane] = acc[b][q];
        acc[b][q] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    lds_barrier();
    if (wave < 2) {
      const int b = wave;
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        f32x4 sum = s_red[0][b][q][lane];
#pragma unroll
        for (int v = 1; v < 4; ++v) sum += s_red[v][b][q][lane];
        // pair r = 16 q + li, output rows 4 * lg + i of block b
        const int r = 16 * q + li;
        if (r >= rows) continue;
        if (kGated) {
          // block 0 holds the gate rows, block 1 the up rows of the same j:
          // wave 0 reads the up partials as well and writes u
          if (b == 1) continue;
          f32x4 up = s_red[0][1][q][lane];
#pragma unroll
          for (int v = 1; v < 4; ++v) up += s_red[v][1][q][lane];
          bf16x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float g = bf16r(silu(bf16r(sum[i])));
            o[i] = static_cast<__bf16>(bf16r(up[i]) * g);
          }
          *reinterpret_cast<bf16x4*>(p.out + int64_t(start + r) * p.out_stride + 16 * ct +
                                     4 * lg) = o;
        } else {
          const int pair = p.sorted[start + r];
          const float wt = p.wts[pair];
          bf16x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = static_cast<__bf16>(bf16r(sum[i]) * wt);
          if (p.fsum != nullptr) {
            __bf16* fo = p.fsum + int64_t(pair / p.topk) * p.fsum_stride + 32 * ct + 16 * b + 4 * lg;
            add_bf16x2(fo, o[0], o[1]);
            add_bf16x2(fo + 2, o[2], o[3]);
          } else {
            *reinterpret_cast<bf16x4*>(p.out + int64_t(pair) * p.out_stride + 32 * ct + 16 * b +
                                       4 * lg) = o;
          }
        }
      }
    }
    // the buffer is next written by the DMA of a later stage, issued after
    // a barrier that every wave reaches only after reading it here
  }
}

// ============================================================================
// final sum over each token's experts
// ============================================================================
struct ReduceParams {
  const __bf16* yw;   // [M * topk, K]
  __bf16* out;
  int64_t s_out;
  int64_t M;
  int K, topk;
};

// One thread per 8 consecutive outputs of a token: the running bf16 sum over
// slots 0..topk-1 (ascending experts), rounded after every add like the
// reference's final_out += (reference.py:35).
__global__ void __launch_bounds__(256) fm_reduce_kernel(const ReduceParams p) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int per = p.K / 8;
  if (i >= p.M * per) return;
  const int64_t t = i / per;
  const int k = int(i % per) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const __bf16* y = p.yw + t * p.topk * int64_t(p.K) + k;
  for (int j = 0; j < p.topk; ++j) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(y + int64_t(j) * p.K);
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = bf16r(acc[c] + static_cast<float>(v[c]));
  }
  bf16x8 o;
#pragma unroll
  for (int c = 0; c < 8; ++c) o[c] = static_cast<__bf16>(acc[c]);
  *reinterpret_cast<bf16x8*>(p.out + t * p.s_out + k) = o;
}

int forward(const fm_args* a, hipStream_t stream, void* const* events, uint32_t* launched) {
  const int rc = validate(a);
  if (rc != FM_OK) return rc;
  if (a->M == 0) return FM_OK;
  const Plan pl = make_plan(a);
  if (a->workspace == nullptr || a->workspace_bytes < pl.bytes) return FM_EWORKSPACE;
  // Launches kernel k (FM_KERNEL_*). With the caller's events, through
  // hipExtLaunchKernel: events[2k] and events[2k+1] take the dispatch's own
  // start and end timestamps.
  auto run = [&](int k, const void* fn, dim3 grid, dim3 block, void** kargs) -> bool {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (events != nullptr) {
      e0 = static_cast<hipEvent_t>(events[2 * k]);
      e1 = static_cast<hipEvent_t>(events[2 * k + 1]);
    }
    const hipError_t err =
        (e0 != nullptr || e1 != nullptr)
            ? hipExtLaunchKernel(fn, grid, block, kargs, 0, stream, e0, e1, 0)
            : hipLaunchKernel(fn, grid, block, kargs, 0, stream);
    if (err != hipSuccess || hipGetLastError() != hipSuccess) return false;
    if (launched != nullptr) *launched |= 1u << k;
    return true;
  };
  auto fn = [](auto kernel) { return reinterpret_cast<const void*>(kernel); };
  uint8_t* ws = static_cast<uint8_t*>(a->workspace);
  int32_t* ids = reinterpret_cast<int32_t*>(ws + pl.ids_off);
  float* wts = reinterpret_cast<float*>(ws + pl.wts_off);
  int32_t* eoff = reinterpret_cast<int32_t*>(ws + pl.eoff_off);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + pl.sorted_off);
  int32_t* tiles = reinterpret_cast<int32_t*>(ws + pl.tiles_off);
  __bf16* inter = reinterpret_cast<__bf16*>(ws + pl.inter_off);
  __bf16* yw = reinterpret_cast<__bf16*>(ws + pl.y_off);

  RouteParams rp{};
  rp.score = static_cast<const __bf16*>(a->score);
  rp.s_score = a->s_score;
  rp.ids = ids;
  rp.wts = wts;
  rp.M = a->M;
  rp.E = int(a->E);
  rp.topk = int(a->topk);
  rp.renormalize = a->renormalize ? 1 : 0;
  // With at most two experts per token, the down GEMM of streamed tiles adds
  // into the output itself and the routing launch clears it: no final-sum
  // launch.
  const bool streamed = !pl.large && a->N % kStK == 0;  // (K % 256 == 0 always holds)
  const bool fsum = streamed && a->topk <= 2 && (a->flags & FM_FLAG_ORDERED_SUM) == 0;
  if (fsum) {
    rp.zero_out = static_cast<__bf16*>(a->out);
    rp.s_out = a->s_out;
    rp.K = int(a->K);
  }
  PlanParams pp{};
  pp.ids = ids;
  pp.eoff = eoff;
  pp.sorted = sorted;
  pp.tiles = tiles;
  pp.P = pl.P;
  pp.E = int(a->E);
  pp.tile_rows = pl.tile_rows;
  if (a->M <= kFusedRouteTokens) {  // one launch, reported as the plan's
    void* ka[] = {&rp, &pp};
    if (!run(FM_KERNEL_PLAN, fn(fm_route_plan_kernel), dim3(1), dim3(1024), ka)) return FM_EHIP;
  } else {
    void* kr[] = {&rp};
    if (!run(FM_KERNEL_ROUTE, fn(fm_route_kernel), dim3(unsigned((a->M + 3) / 4)), dim3(256), kr))
      return FM_EHIP;
    void* kp[] = {&pp};
    if (!run(FM_KERNEL_PLAN, fn(fm_plan_kernel), dim3(1), dim3(1024), kp)) return FM_EHIP;
  }

  GemmParams g1{};
  g1.a = static_cast<const __bf16*>(a->hidden);
  g1.a_stride = a->s_hidden;
  g1.w = static_cast<const __bf16*>(a->w1);
  g1.w_estride = 2 * a->N * a->K;
  g1.sorted = sorted;
  g1.tiles = tiles;
  g1.wts = wts;
  g1.out = inter;
  g1.out_stride = a->N;
  g1.kin = int(a->K);
  g1.nout = int(a->N);
  g1.topk = int(a->topk);
  GemmParams g2 = g1;
  g2.a = inter;
  g2.a_stride = a->N;
  g2.w = static_cast<const __bf16*>(a->w2);
  g2.w_estride = a->K * a->N;
  g2.out = yw;
  g2.out_stride = a->K;
  g2.kin = int(a->N);
  g2.nout = int(a->K);
  if (pl.large) {
    g1.col_tiles = int(a->N / (kLargeCols / 2));
    g2.col_tiles = int(a->K / kLargeCols);
  } else {
    g1.col_tiles = int(a->N / 16);
    g2.col_tiles = int(a->K / 32);
  }
  // small tiles stream their weights through LDS when both reductions are
  // whole 256-wide stages, else straight into registers
  if (fsum) {
    g2.fsum = static_cast<__bf16*>(a->out);
    g2.fsum_stride = a->s_out;
  }
  g1.ct_per_wg = g2.ct_per_wg = 1;
  // (MI355X: 256 CUs, one large or big work-group each)
  const double pairs_per_expert = double(pl.P) / double(a->E);
  for (GemmParams* g : {&g1, &g2})
    g->xcd_grid = pl.large && pairs_per_expert < 2.0 * pl.tile_rows &&
                  pl.max_tiles * g->col_tiles > 256;
  if (streamed) {
    // a streaming work-group runs several column tiles in one pipeline, so its
    // start (tile table -> pair list -> first DMA) is paid once per
    // several: about 1024 work-groups per launch, whole column tiles each
    for (GemmParams* g : {&g1, &g2}) {
      int c = 1;
      while (c * 2 <= g->col_tiles && pl.max_tiles * (g->col_tiles / (c * 2)) >= 1024) c *= 2;
      g->ct_per_wg = c;
    }
  }
  auto grid_of = [&](const GemmParams& g) {
    if (pl.large)  // xcd_item: each XCD has up to ceil(tiles / 4) x ceil(col_tiles / 2) items
      return unsigned(kXcds * ((pl.max_tiles + kXcdTileGroups - 1) / kXcdTileGroups) *
                      ((g.col_tiles + kXcdColGroups - 1) / kXcdColGroups));
    return unsigned(pl.max_tiles * ((g.col_tiles + g.ct_per_wg - 1) / g.ct_per_wg));
  };
  const unsigned grid1 = grid_of(g1);
  const unsigned grid2 = grid_of(g2);
  // the GEMM kernel of this plan, gated (gate-up) or not (down)
  auto gemm = [&](auto gated) -> const void* {
    constexpr bool G = decltype(gated)::value;
    if (pl.big) return fn(fm_gemm_big_kernel<G>);
    if (pl.large) return fn(fm_gemm_kernel<G>);
    if (streamed)
      return pl.pb == 1 ? fn(fm_stream_kernel<G, 1>)
                        : pl.pb == 2 ? fn(fm_stream_kernel<G, 2>) : fn(fm_stream_kernel<G, 4>);
    return pl.pb == 1 ? fn(fm_skinny_kernel<G, 1>) : fn(fm_skinny_kernel<G, 2>);
  };
  const dim3 gemm_block(pl.big ? 512 : 256);
  void* k1[] = {&g1};
  if (!run(FM_KERNEL_GATEUP, gemm(std::true_type{}), dim3(grid1), gemm_block, k1)) return FM_EHIP;
  void* k2[] = {&g2};
  if (!run(FM_KERNEL_DOWN, gemm(std::false_type{}), dim3(grid2), gemm_block, k2)) return FM_EHIP;

  if (fsum) return FM_OK;
  ReduceParams rd{};
  rd.yw = yw;
  rd.out = static_cast<__bf16*>(a->out);
  rd.s_out = a->s_out;
  rd.M = a->M;
  rd.K = int(a->K);
  rd.topk = int(a->topk);
  const int64_t threads = a->M * (a->K / 8);
  void* kd[] = {&rd};
  return run(FM_KERNEL_REDUCE, fn(fm_reduce_kernel), dim3(unsigned((threads + 255) / 256)),
             dim3(256), kd) ? FM_OK : FM_EHIP;
}

}  // namespace

extern "C" {

int fm_abi_version(void) { return FM_ABI_VERSION; }

const char* fm_strerror(int code) {
  switch (code) {
    case FM_OK: return "ok";
    case FM_EINVAL: return "invalid argument (null pointer, size, stride, alignment or flags)";
    case FM_EUNSUPPORTED:
      return "unsupported shape (needs K % 256 == 0, N % 128 == 0, E <= 256, topk <= 32 and "
             "sizes within 32-bit offsets)";
    case FM_EWORKSPACE: return "workspace missing or too small";
    case FM_EHIP: return "HIP runtime error";
    default: return "unknown error";
  }
}

int fm_workspace_bytes(const fm_args* a, size_t* out_bytes) {
  if (out_bytes == nullptr) return FM_EINVAL;
  const int rc = validate(a);
  if (rc != FM_OK) return rc;
  *out_bytes = a->M == 0 ? 0 : make_plan(a).bytes;
  return FM_OK;
}

int fm_forward(const fm_args* a, void* hip_stream) {
  return forward(a, static_cast<hipStream_t>(hip_stream), nullptr, nullptr);
}

int fm_forward_events(const fm_args* a, void* hip_stream, void* const* events,
                      uint32_t* launched) {
  if (launched != nullptr) *launched = 0u;
  return forward(a, static_cast<hipStream_t>(hip_stream), events, launched);
}

}  // extern "C"
