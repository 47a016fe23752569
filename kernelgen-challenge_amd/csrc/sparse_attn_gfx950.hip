// sparse_attn_gfx950.hip -- MI355X (gfx950, CDNA4) kernels and C-ABI for
// top-k sparse attention with an attention sink, h = 16, d = 512, bf16 I/O.
//
// Math (track-01/reference/reference.py:24-40): for each query (b, m) and
// head h, s_t = scale * q[h] . kv[idx_t]; o[h] = sum_t softmax([s, sink[h]])_t
// * kv[idx_t] with the sink column dropped; o cast to bf16 (round to nearest
// even). -1 slots are excluded (track-01/submission.py:313-322); duplicated
// indices count with multiplicity (gather semantics, reference.py:28).
//
// Scores live in the log2 domain (scale * log2 e folded in, exp2) and the sink
// is folded last as m_tot = max(m, sink), l_tot = 2^(m - m_tot) l +
// 2^(sink - m_tot), which equals the reference's softmax over [s, sink]
// (track-01/notes.md:32-41).
//
// Kernels
// -------
// sa_tile_index_kernel  one work-group per tile of 8 consecutive queries of a
//   batch: counts every valid index of the tile's queries in an LDS table
//   (one byte per query), writes the row union in ascending order (32-bit
//   byte offsets) with an fp16 log2 multiplicity per (query, row), and marks
//   the tile "shared" when the shared-row kernel would spend less CU time on
//   it than the per-query kernel on its queries, else "per query". With long
//   caches and short queries the mode comes first, from a bitmap of the
//   tile's rows, and only shared tiles are counted.
// sa_order_kernel  one work-group: the tile order (a counting sort by
//   descending step count, so the longest tiles are launched first) where no
//   per-query launch makes it (index plans, and the ordered short-query
//   launch).
// sa_fwd_tile_kernel  one work-group per shared tile (128 query-head
//   columns): gathers each union row once (LDS-DMA, 1 KiB per instruction),
//   S^T = K . Q^T with each wave owning two queries, P through LDS, O += P . V
//   with each wave owning a quarter of d; v_mfma_f32_32x32x16_bf16; the
//   softmax of one 32-row half runs between the MFMAs of the next. A fixed
//   per-column reference replaces rescaling; a tile whose scores jump above
//   it runs its queries per query in place. Work-group i runs entry i of the
//   tile order, or (short-query plans) one work-group per CU walks the
//   tiles' modes and runs the shared ones.
// sa_fwd_query_kernel  one work-group (4 wave64s) per (query, topk part);
//   in a shared-row plan (before the shared-row kernel) one per tile, which
//   runs the queries of a per-query tile in turn, and work-group 0 makes the
//   tile order. Compacts the part's valid indices into LDS,
//   then streams steps of 32 gathered rows through a ring of LDS buffers
//   filled by LDS-DMA (4 buffers, or 2 and two work-groups per CU when the
//   launch has at least two per CU). S^T = K . Q^T with v_mfma_f32_16x16x32_bf16 (wave w:
//   the step's rows 8w.., 16 heads, K = d = 512, Q^T resident in registers);
//   online softmax with a per-head max across the waves through LDS;
//   O += P . V with the same MFMA (wave w: d columns 128w..), its V operands
//   read from the same LDS rows by ds_read_b64_tr_b16 transposing reads.
//   Writes bf16 o, or per-part (max, sum, unnormalised O) for
//   sa_combine_kernel.
// sa_fwd_wave_kernel  unsplit queries with topk <= 384 (per-query tiles of
//   shared-row plans, or every query of a per-query plan): one wave64 work-
//   group per two queries, a stream of 16-row steps through the wave's own
//   2-deep LDS-DMA ring, no barrier. S^T = K . Q^T (16x16x32 MFMA, Q^T as
//   an AGPR operand), the softmax inside the wave, O += P . V with
//   v_mfma_f32_16x16x16_bf16 taking P from the S^T accumulators. Each
//   query's rows are sorted ascending when a batch's kv exceeds an XCD's L2.
// sa_combine_kernel  merges the topk parts of one (query, head), folds the
//   sink and stores bf16.
// sa_merge_kernel  merges caller-supplied (o, lse) partials (sa_merge).
// sa_pad_heads_kernel, sa_unpad_heads_kernel  calls with 1, 2, 4 or 8 heads
//   run on a 16-head copy in the workspace (q zero-padded in, o copied out).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "sa_plan.h"
#include "sparse_attn.h"

namespace {

using sa::kDim;
using sa::kHeads;
using sa::kMetaInts;
using sa::kModeShared;
using sa::kTileRows;

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRowBytes = kDim * 2;           // one kv row, 1 KiB
constexpr int kRowStride = kRowBytes + 32;    // padded LDS row pitch (bytes)
constexpr int kListCap = 2048;                // compacted slots per batch
constexpr int kSlotsPerThread = kListCap / kThreads;
constexpr int kRowsPerWave = kTileRows / kWaves;  // 16
constexpr int kDPerWave = kDim / kWaves;          // 128 output columns
constexpr int kDBlocks = kDPerWave / 16;          // 8 MFMA column blocks
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Lazy rescaling: the running reference max of a softmax column moves only
// when a tile's max exceeds it by more than this (log2 units), so exp2(s - m)
// stays below 2^8 and the accumulators are rescaled rarely.
constexpr float kRescaleLog2 = 8.f;
// Shared tiles never rescale O: scores may exceed a column's fixed reference
// by up to this (log2 units; weights <= 255 * 2^24 stay far from fp32 and
// bf16 overflow). A larger jump makes the tile run its queries per query
// (online rescale) instead.
constexpr float kTileMaxJump = 24.f;

constexpr int kTQ = sa::kTileQueries;       // queries per shared tile
// A tile is shared when the shared-row kernel's CU time for it is below the
// per-query kernel's for its queries, with a margin for the per-query side.
// Measured on MI355X (CU time, nanoseconds): a shared tile costs about
// 10 000 (start and epilogue) plus 6.6 per dense (tile query x union row)
// pair, all 8 columns counted whatever the tile holds (causal prefill). The
// queries of per-query tiles run in the per-query launch that follows the
// shared-row kernel, two work-groups per CU, whose starts and ends overlap
// each other's gathers: a query costs about 2 100 plus 27 per valid slot
// (topk 128 at kv_len 1 024 - 16 384: 5.3-5.9 us per query; topk 640 at
// kv_len 20 480: 19.2 us).
// When every tile starts at once (between half as many tiles as CUs and as
// many), the per-query launch's time adds to the slowest tile's instead of
// filling in behind other tiles, and its work-groups have a CU each: a query
// is priced at 4 900 plus 35 per slot. (At the lower price high locality's
// longest tiles went per query and the call took 134 us instead of 116.)
constexpr int64_t kSharedTileNs = 10000;
constexpr int64_t kSharedPairNs10 = 66;   // x 10
constexpr int64_t kQueryUnitNs = 2100;
constexpr int64_t kQuerySlotNs = 27;
constexpr int64_t kPlacedQueryUnitNs = 4900;
constexpr int64_t kPlacedQuerySlotNs = 35;
constexpr int64_t kSharedMarginPct = 85;  // shared only below 85 % of per-query

// The mode rule: shared when the tile's shared-row time is below
// kSharedMarginPct % of its queries' per-query time.
__host__ __device__ constexpr bool shared_is_cheaper(int64_t n_union, int64_t n_valid,
                                                    int64_t queries, bool placed_regime) {
  return 100 * (10 * kSharedTileNs + kSharedPairNs10 * kTQ * n_union) <=
         kSharedMarginPct * 10 *
             ((placed_regime ? kPlacedQueryUnitNs : kQueryUnitNs) * queries +
              (placed_regime ? kPlacedQuerySlotNs : kQuerySlotNs) * n_valid);
}

// An order entry of the tile order kernel is (key << kOrderTileBits) | tile:
// key 0 for a per-query tile, else 1 + its step count, so the shared-row
// kernel learns its tile and step count from one load. A plan has at most
// b * m / 4 <= 2^22 tiles.
constexpr int kOrderTileBits = 22;
static_assert(sa::kMaxUnits / (sa::kTileQueries / 2) <= (int64_t(1) << kOrderTileBits),
              "tile ids fit the order entry");

static_assert(kListCap % kThreads == 0, "compaction split");
static_assert(kRowsPerWave == 16, "one 16-row MFMA block per wave");
static_assert(kTQ == 2 * kWaves && kTileRows == 64, "shared tile wave layout");

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

// Arguments of the tile order (see make_order).
struct OrderParams {
  const int32_t* meta;
  int32_t* order;
  int ntiles;
  int cus;  // compute units of the device
};

struct FwdParams {
  const __bf16* q;
  const __bf16* kv;
  const float* sink;
  const int32_t* idx;
  __bf16* o;
  float* part;          // [units * nsplit] x (ml[32] + O[16*512]) when split
  int32_t* err;
  int64_t m, kv_len, topk;
  int64_t sq_b, sq_m, sq_h;
  int64_t skv_b, skv_n;
  int64_t si_b, si_m;
  int64_t so_b, so_m, so_h;
  float scale_log2;     // scale * log2(e)
  float* lse;           // fp32 [b, m, h] or null
  int64_t sl_b, sl_m, sl_h;
  int nsplit;
  int64_t split_len;
  int64_t nblocks;      // grid size (units * nsplit)
  // Shared-row plans (nsplit = 1): the index kernel's tile meta (the launch
  // runs the queries of per-query tiles) and the tile order to make, if any.
  const int32_t* meta;
  int64_t tiles_per_b;
  OrderParams ord;
  // sa_fwd_wave_kernel: walk each query's rows in ascending order (a batch's
  // kv larger than an XCD's L2)
  int sort_wave;
};

struct IndexParams {
  const int32_t* idx;
  int32_t* err;
  int32_t* meta;        // [ntiles][kMetaInts]
  uint32_t* row_off;    // [ntiles][cap] byte offsets of the union rows in the batch's kv
  _Float16* lcnt;       // [ntiles][cap / 64][kTQ][64] log2 multiplicities (-inf: absent)
  int64_t m, kv_len, topk;
  int64_t si_b, si_m;
  int64_t skv_n;        // kv row stride (elements)
  int64_t tiles_per_b, cap;
  int force;            // shared mode whenever the counts fit
  int vec4;             // indices readable as int4 (aligned base, strides and topk)
  int placed_regime;    // every tile starts at once (see kPlacedQueryUnitNs)
};

struct TileParams {
  const __bf16* q;
  const __bf16* kv;
  const float* sink;
  __bf16* o;
  const int32_t* order; // work-group i runs entry order[i]
  const uint32_t* row_off;
  const _Float16* lcnt;
  int64_t m, cap, tiles_per_b;
  int64_t sq_b, sq_m, sq_h;
  int64_t skv_b, skv_n;
  int64_t so_b, so_m, so_h;
  float scale_log2;
  float* lse;           // fp32 [b, m, h] or null
  int64_t sl_b, sl_m, sl_h;
  int64_t ntiles;
  FwdParams fwd;        // arguments of the queries of aborted tiles (nsplit = 1)
  // Placed launch (no order kernel): work-group i runs tile xcd_tile(i), its
  // step count and mode read from the index kernel's meta.
  int placed;
  const int32_t* meta;
};

struct CombineParams {
  const float* part;
  const float* sink;
  __bf16* o;
  float* lse;           // fp32 [b, m, h] or null
  int64_t m;
  int64_t so_b, so_m, so_h;
  int64_t sl_b, sl_m, sl_h;
  int nsplit;
};

struct MergeParams {
  const __bf16* o_parts;
  const float* lse_parts;
  const float* sink;    // null: no sink
  __bf16* o;
  float* lse;
  int64_t n, b, m, h, d;
  int64_t sop_n, sop_b, sop_m, sop_h;
  int64_t slp_n, slp_b, slp_m, slp_h;
  int64_t so_b, so_m, so_h;
  int64_t sl_b, sl_m, sl_h;
};

constexpr int64_t kPartFloats =
    (sa::kPartialMLBytes + sa::kPartialOBytes) / sizeof(float);

__device__ __forceinline__ f32x4 mfma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_bf16 accumulating in AGPRs, issued as inline assembly
// so that the compiler's own MFMAs in the same kernel keep their accumulators
// in VGPRs (the library is built with -amdgpu-mfma-vgpr-form): the shared-row
// kernel needs all 256 AGPRs for O and 32 VGPRs for S at the same time.
// Hazards the compiler cannot see:
//  * a VALU write of an A/B operand register needs 2 wait states before the
//    MFMA reads it: s_nop 1 gives them;
//  * back-to-back accumulation into the same registers needs none;
//  * AGPR reads of the results (v_accvgpr_read) need the MFMA's 8 passes plus
//    3: mfma_agpr_drain() gives 16 wait states.
__device__ __forceinline__ void mfma_agpr(f32x16& c, bf16x8 a, bf16x8 b) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
      : "+a"(c)
      : "v"(a), "v"(b));
}

// v_mfma_f32_16x16x32_bf16 accumulating in VGPRs with its B operand in
// AGPRs (an operand that lives in AGPRs for good, such as a resident Q^T,
// then takes no VGPRs). The same hazards; the VALU reads of the result wait
// for mfma_agpr_drain().
__device__ __forceinline__ void mfma32_bagpr(f32x4& c, bf16x8 a, const bf16x8& b) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
      : "+v"(c)
      : "v"(a), "a"(b));
}

__device__ __forceinline__ f32x4 mfma_16x16x16(bf16x4 a, bf16x4 b, f32x4 c) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                  __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

__device__ __forceinline__ void mfma_agpr_drain() {
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
}

// Sink fold in the log2 domain (track-01/notes.md:32-41): m, l are the max
// (or any reference at or below it; -inf when there is no valid slot) and the
// sum of 2^(x - m) over the valid slots, sink2 = sink * log2 e. Returns the
// factor that turns the unnormalised output into o, and the natural-log
// lse = ln(sum exp(s) + exp(sink)). No mass at all (no slot, sink = -inf):
// factor 0 (o = 0) and lse = -inf.
__device__ __forceinline__ float sink_fold(float m, float l, float sink2, float& lse) {
  const float mt = fmaxf(m, sink2);
  if (mt == -INFINITY) {
    lse = -INFINITY;
    return 0.f;
  }
  const float a = exp2f(m - mt);  // 0 when m = -inf
  const float den = a * l + exp2f(sink2 - mt);
  lse = (mt + log2f(den)) * kLn2;
  return a / den;
}

// Reports an index outside [-1, kv_len): *err = 1 as a system-scope store
// (a vector store), so the word may also be mapped pinned host memory that
// the host reads without synchronizing. Every writer stores the same value.
__device__ __forceinline__ void flag_bad_index(int32_t* err) {
  __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane j supplies the address
// of 4 consecutive bf16 (row j/4, columns 4*(j%4)..+3 of a 4 x 16 block) and
// receives column j of that block (4 values, one per row).
__device__ __forceinline__ bf16x4 lds_read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)((lds_u8_t*)(p)));
}

// LDS-DMA issued from inline assembly: every lane moves 16 bytes from its own
// global address to lds + lane * 16 (`lds` wave-uniform). Used by pipelines
// that read one LDS buffer while gathering into another: the compiler does
// not see this as an LDS write, so it does not wait for the gather before
// every LDS read. The caller must wait (vmcnt = 0, e.g. dma_barrier()) before
// any wave reads the destination. The LDS address goes in M0 through the
// "{m0}" operand constraint, so the compiler writes M0 itself and knows what
// it holds; s_nop 0 gives the wait state between that SALU write and the
// load that reads M0.
__device__ __forceinline__ void lds_dma16_async(const void* gsrc, void* lds) {
  const uint32_t lds_addr =
      __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>((lds_u8_t*)(lds))));
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(gsrc), "{m0}"(lds_addr)
      : "memory");
}

// LDS-DMA of one 1 KiB row at a wave-uniform address: SGPR base `row` plus the
// 32-bit lane offset 16 * lane, into LDS bytes lds_addr + 16 * lane. Measured
// on gfx950, this form blocks the issuing wave for about 27 cycles against 46
// for the same transfer with a 64-bit per-lane address.
// M0 as in lds_dma16_async.
__device__ __forceinline__ void lds_dma_row(const void* row, uint32_t lane_off, uint32_t lds_addr) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(lane_off), "s"(row), "{m0}"(lds_addr)
      : "memory");
}

// Work-group barrier that orders LDS traffic only: waits for this wave's LDS
// reads and writes (lgkmcnt = 0) but not for outstanding global loads, so a
// prefetch issued earlier keeps flying across it. (__syncthreads() would also
// drain every global load in flight.)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt = max, expcnt = max, lgkmcnt = 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Barrier after which this wave's LDS-DMA transfers are complete as well.
__device__ __forceinline__ void dma_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Reductions over lanes n, n + 16, n + 32, n + 48 (the four lane rows of a
// wave64). v_permlane16_swap with both operands x gives lane n the values of
// lanes n and n ^ 16 (as its two results), v_permlane32_swap those of n and
// n ^ 32: two VALU instructions per level, against __shfl_xor's
// ds_bpermute (an LDS round trip plus its index arithmetic). The sums add in
// the same order as a butterfly: (x[n] + x[n^16]) + (x[n^32] + x[n^48]).
__device__ __forceinline__ float wave_max16(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float wave_sum16(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ============================================================================
// per-query kernel
// ============================================================================
// The rows of a part stream through a ring of kRing LDS buffers of kQRows
// rows each, filled by LDS-DMA (one 1 KiB row per wave instruction). While
// the work-group computes on one buffer, the gathers of the next kRing - 1
// steps are in flight.
//  * kRing = 4 (96 KiB in flight per work-group, 145 KiB of LDS: one
//    work-group per CU): a short part (decode) has its whole gather issued
//    within its first steps, and a long one keeps enough bytes in flight per
//    CU to run at the random-row gather rate.
//  * kRing = 2 (77 KiB of LDS: two work-groups per CU), for launches with
//    several work-groups per CU: one work-group's start (index load,
//    compaction, first gathers) and end overlap the other's gathers.
constexpr int kQRows = 32;
constexpr int kQRowsPerWave = kQRows / kWaves;  // rows of a step each wave gathers
static_assert(kQRowsPerWave == 8, "the vmcnt waits of the ring");

template <int kRing>
struct QuerySmemT {
  uint8_t tile[kRing][kQRows * kRowStride];
  int32_t list[kListCap];
  __bf16 p[kHeads * kQRows];
  float red[kWaves][kHeads];
  int cnt[kWaves];
  int qstart[kTQ + 1];  // query_stream: query j's entries of `list` start here
};
using QuerySmem = QuerySmemT<4>;
static_assert(sizeof(QuerySmemT<2>) <= 80 * 1024, "two ring-2 work-groups per CU");

// Waits until at most the gathers of `later` (0..2) steps issued after the
// current one are outstanding: this wave's rows of the current step are in
// LDS. Loads return in order, and each step is kQRowsPerWave loads per wave.
__device__ __forceinline__ void wait_ring(int later) {
  if (later >= 2)
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if (later == 1)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Per-query kernel state of one (query, part) for this lane: the running max
// (log2 domain) and this lane's share of the running sum of head n, O, and
// Q^T as the B operand of S^T = K . Q^T (lane (n, g) holds head n,
// d = 32s + 8g .. 32s + 8g + 7 for k-step s).
struct QueryState {
  float m_run;
  float l_run;
  f32x4 oacc[kDBlocks];
  bf16x8 qf[kDim / 32];
};

__device__ __forceinline__ void query_state_reset(QueryState& st) {
  st.m_run = -INFINITY;
  st.l_run = 0.f;
#pragma unroll
  for (int i = 0; i < kDBlocks; ++i) st.oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// Issues the loads of query (bi, mi)'s Q^T into st.qf.
__device__ __forceinline__ void query_load_q(const FwdParams& p, int64_t bi, int64_t mi,
                                             QueryState& st) {
  const int lane = threadIdx.x & 63;
  const __bf16* qrow = p.q + bi * p.sq_b + mi * p.sq_m + int64_t(lane & 15) * p.sq_h +
                       8 * (lane >> 4);
#pragma unroll
  for (int s = 0; s < kDim / 32; ++s) st.qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
}

// One step of the per-query kernel over the 32 rows in LDS buffer `tb`, of
// which the first `nrows` are valid (at least one): S^T for this wave's 8
// rows, the online softmax (per-head max across the waves through LDS), and
// O += P . V. When `dma`, this wave's 8 gathers of a later step (rows
// readlane(rv, i) of `kvb`, into LDS at lbase + i * kRowStride) ride between
// the S^T MFMAs; with kByteOffsets, rv holds the rows' 32-bit byte offsets
// in `kvb` instead (one scalar add per address instead of a 64-bit
// multiply). `after_s` runs once S^T is done (Q^T is no longer read).
template <int kRing, bool kByteOffsets = false, typename AfterS>
__device__ __forceinline__ void query_step(const FwdParams& p, QuerySmemT<kRing>& sm,
                                           const uint8_t* tb, bool dma, int rv, uint32_t lbase,
                                           const uint8_t* kvb, int64_t row_bytes, int nrows,
                                           QueryState& st, AfterS after_s) {
  auto& s_p = sm.p;
  auto& s_red = sm.red;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15;   // MFMA column lane: head (S^T, P) or d (O)
  const int g = lane >> 4;   // MFMA k-group
  float& m_run = st.m_run;
  float& l_run = st.l_run;
  auto& oacc = st.oacc;
  const auto& qf = st.qf;

  // ---- S^T = K . Q^T for this wave's 8 rows ----------------------------------
  // MFMA rows 8..15 repeat rows 0..7 (the A operand reads row n & 7). The K
  // fragments are read 3 MFMAs ahead; the 8 row gathers of the later step
  // ride between the MFMAs (one after every second), where their issue cost
  // overlaps the MFMA chain.
  f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
  {
    const uint8_t* krow = tb + (wave * kQRowsPerWave + (n & 7)) * kRowStride + 16 * g;
    auto s_chain = [&](auto with_dma) {
      bf16x8 kf[4];
#pragma unroll
      for (int s = 0; s < 3; ++s) kf[s] = *reinterpret_cast<const bf16x8*>(krow + 64 * s);
#pragma unroll
      for (int s = 0; s < kDim / 32; ++s) {
        if (s + 3 < kDim / 32)
          kf[(s + 3) & 3] = *reinterpret_cast<const bf16x8*>(krow + 64 * (s + 3));
        sacc = mfma_16x16x32(kf[s & 3], qf[s], sacc);
        if constexpr (decltype(with_dma)::value) {
          if (s & 1) {
            const int i = s >> 1;
            const int row = __builtin_amdgcn_readlane(rv, i);
            const uint8_t* src =
                kByteOffsets ? kvb + uint32_t(row) : kvb + int64_t(row) * row_bytes;
            lds_dma_row(src, 16 * lane, lbase + uint32_t(i * kRowStride));
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the interleave
      }
    };
    static_assert(kDim / 32 == 2 * kQRowsPerWave, "one gather per two S^T MFMAs");
    if (dma)
      s_chain(std::true_type{});
    else
      s_chain(std::false_type{});
  }
  after_s();
  // lane (n, g) now holds S[head n][row 8w + 4g + j], j = 0..3; lanes with
  // g >= 2 hold the repeated rows and drop them

  // ---- online softmax ------------------------------------------------------
  const int rbase = wave * kQRowsPerWave + 4 * g;  // row within the step
  float sv[4];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sv[j] = (g < 2 && rbase + j < nrows) ? sacc[j] * p.scale_log2 : -INFINITY;
    mx = fmaxf(mx, sv[j]);
  }
  mx = wave_max16(mx);
  if (g == 0) s_red[wave][n] = mx;
  lds_barrier();
  // finite: the step's first row is valid (wave 0)
  const float mstep = fmaxf(fmaxf(s_red[0][n], s_red[1][n]), fmaxf(s_red[2][n], s_red[3][n]));
  float alpha = 1.f;
  if (mstep > m_run + kRescaleLog2) {
    // v_exp_f32 as is: exp2f adds a rescale for results below 2^-126, which
    // are negligible next to the running sum (at least 1)
    alpha = m_run == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - mstep);
    m_run = mstep;
  }
  float psum = 0.f;
  bf16x4 pb;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float pj = __builtin_amdgcn_exp2f(sv[j] - m_run);
    psum += pj;
    pb[j] = static_cast<__bf16>(pj);
  }
  l_run = l_run * alpha + psum;
  if (g < 2) *reinterpret_cast<bf16x4*>(&s_p[n * kQRows + wave * kQRowsPerWave + 4 * g]) = pb;
  if (__any(alpha != 1.f)) {
    float aj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) aj[j] = __shfl(alpha, 4 * g + j);
#pragma unroll
    for (int blk = 0; blk < kDBlocks; ++blk)
#pragma unroll
      for (int j = 0; j < 4; ++j) oacc[blk][j] *= aj[j];
  }
  lds_barrier();  // P of every wave is in LDS

  // ---- O[:, 128w .. 128w+127] += P . V over the step's 32 rows ---------------
  {
    const bf16x8 pf = *reinterpret_cast<const bf16x8*>(&s_p[n * kQRows + 8 * g]);
    const uint8_t* vb =
        tb + (8 * g + (n >> 2)) * kRowStride + (wave * kDPerWave + 4 * (n & 3)) * 2;
#pragma unroll
    for (int blk = 0; blk < kDBlocks; ++blk) {
      const bf16x4 v0 = lds_read_tr16(vb + blk * 32);
      const bf16x4 v1 = lds_read_tr16(vb + 4 * kRowStride + blk * 32);
      const bf16x8 vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      oacc[blk] = mfma_16x16x32(pf, vf, oacc[blk]);
    }
  }
}

// The end of a (query, part) unit: the running sum across the waves, then
// bf16 o (and lse) with the sink folded in, or this part's (max, sum,
// unnormalised O) for the combine kernel when the query is split. Every wave
// is past its LDS accesses only after the work-group's final barrier here.
template <int kRing>
__device__ __forceinline__ void query_epilogue(const FwdParams& p, QuerySmemT<kRing>& sm,
                                               int64_t unit, int64_t bi, int64_t mi,
                                               const QueryState& st) {
  auto& s_red = sm.red;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const float m_run = st.m_run;
  const float l_run = st.l_run;
  const auto& oacc = st.oacc;
  float lw = wave_sum16(l_run);
  __syncthreads();
  if (g == 0) s_red[wave][n] = lw;
  __syncthreads();
  const float l_tot = s_red[0][n] + s_red[1][n] + s_red[2][n] + s_red[3][n];
  const int dcol = wave * kDPerWave + n;

  if (p.nsplit == 1) {
    float lse;
    const float f = sink_fold(m_run, l_tot, p.sink[n] * kLog2e, lse);
    if (p.lse != nullptr && wave == 0 && g == 0)
      p.lse[bi * p.sl_b + mi * p.sl_m + int64_t(n) * p.sl_h] = lse;
    float fj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fj[j] = __shfl(f, 4 * g + j);
    __bf16* ob = p.o + bi * p.so_b + mi * p.so_m;
    // o and the partials are written once and not read again by this launch:
    // nontemporal stores keep them from taking L2 lines from the gathered rows
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      __bf16* orow = ob + int64_t(4 * g + j) * p.so_h + dcol;
#pragma unroll
      for (int blk = 0; blk < kDBlocks; ++blk)
        __builtin_nontemporal_store(static_cast<__bf16>(oacc[blk][j] * fj[j]), &orow[16 * blk]);
    }
  } else {
    float* part = p.part + unit * kPartFloats;
    if (wave == 0 && g == 0) {
      part[n] = m_run;
      part[kHeads + n] = l_tot;
    }
    float* po = part + 2 * kHeads;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int blk = 0; blk < kDBlocks; ++blk)
        __builtin_nontemporal_store(oacc[blk][j], &po[(4 * g + j) * kDim + dcol + 16 * blk]);
  }
}

// Sorts the first kThreads * R entries of the LDS list `s` ascending, in
// place: a bitonic network over kThreads * R keys, R consecutive keys per
// thread. Entries at or past `n` count as +inf, so the n valid entries end up
// in front, sorted; the caller reads no further. Steps whose partner key is
// in the same thread compare registers, steps within a wave exchange them by
// lane shuffles, and the steps across waves (partner distance >= 64 R) go
// through the list itself between barriers. The result is the sorted
// sequence, whatever order the entries came in. Not inlined: inside the
// per-query unit, where Q^T and O are live, the unrolled network made the
// compiler spill scalar registers and use scratch.
template <int R>
__device__ __attribute__((noinline)) void sort_list(int32_t* s, int n) {
  constexpr int N = kThreads * R;
  const int tid = threadIdx.x;
  int v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid * R + r;
    v[r] = i < n ? s[i] : INT32_MAX;
  }
  // the element of key position i keeps the smaller of the pair when the
  // pair's run ascends and i is its lower position, or descends and i is not
  auto keep = [](int mine, int other, int i, int k, int j) {
    const bool up = (i & k) == 0, low = (i & j) == 0;
    return up == low ? min(mine, other) : max(mine, other);
  };
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((r & j) != 0) continue;
          const int i = tid * R + r;
          const int a = v[r], b = v[r | j];
          const bool up = (i & k) == 0;
          v[r] = up ? min(a, b) : max(a, b);
          v[r | j] = up ? max(a, b) : min(a, b);
        }
      } else if (j < 64 * R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int o = __shfl_xor(v[r], j / R);
          v[r] = keep(v[r], o, tid * R + r, k, j);
        }
      } else {
        lds_barrier();  // every wave is past its last read of the list
#pragma unroll
        for (int r = 0; r < R; ++r) s[tid * R + r] = v[r];
        lds_barrier();
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = keep(v[r], s[(tid * R + r) ^ j], tid * R + r, k, j);
      }
    }
  }
  lds_barrier();
#pragma unroll
  for (int r = 0; r < R; ++r) s[tid * R + r] = v[r];
  lds_barrier();
}

// Sorts s[0, n) ascending, as unsigned keys, with one wave (n <= 64 R): a
// bitonic network over 64 R keys, R consecutive keys per lane, padded with
// UINT32_MAX (never a row's byte offset, a multiple of the row size). Steps
// whose partner key is in the same lane compare registers; the others
// exchange keys by lane shuffles. Only s[0, n) is written back, so a list
// that follows in LDS is untouched. Not inlined, for the reason sort_list is
// not.
template <int R>
__device__ __attribute__((noinline)) void sort_list_wave(uint32_t* s, int n) {
  constexpr int N = 64 * R;
  const int lane = threadIdx.x & 63;
  uint32_t v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = lane * R + r;
    v[r] = i < n ? s[i] : UINT32_MAX;
  }
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if ((r & j) != 0) continue;
          const uint32_t a = v[r], b = v[r | j];
          const bool up = ((lane * R + r) & k) == 0;
          v[r] = up ? min(a, b) : max(a, b);
          v[r | j] = up ? max(a, b) : min(a, b);
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t o = uint32_t(__shfl_xor(int(v[r]), j / R));
          const int i = lane * R + r;
          const bool up = (i & k) == 0, low = (i & j) == 0;
          v[r] = up == low ? min(v[r], o) : max(v[r], o);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = lane * R + r;
    if (i < n) s[i] = v[r];
  }
}

// One (query, topk part) unit of the per-query kernel. Leaves every wave past
// its last LDS access of `sm` only after the work-group's final barrier, so a
// following unit may reuse `sm` after one more __syncthreads().
template <int kRing>
__device__ __forceinline__ void query_unit(const FwdParams& p, const int64_t unit,
                                           QuerySmemT<kRing>& sm) {
  constexpr int kQRing = kRing;
  constexpr int kQAhead = kRing - 1;
  static_assert(kQAhead >= 1 && kQAhead <= 3, "wait_ring covers up to 2 later steps");
  auto& s_list = sm.list;
  auto& s_cnt = sm.cnt;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int64_t qid = unit / p.nsplit;
  const int split = int(unit % p.nsplit);
  const int64_t bi = qid / p.m;
  const int64_t mi = qid % p.m;
  const int64_t s_begin = int64_t(split) * p.split_len;
  const int64_t s_end = min(p.topk, s_begin + p.split_len);

  const uint8_t* kvb = reinterpret_cast<const uint8_t*>(p.kv + bi * p.skv_b);
  const int64_t row_bytes = p.skv_n * 2;
  const int32_t* irow = p.idx + bi * p.si_b + mi * p.si_m;
  // LDS address of this wave's first row in ring buffer 0
  const uint32_t lds_rows = __builtin_amdgcn_readfirstlane(uint32_t(
      reinterpret_cast<uintptr_t>((lds_u8_t*)&sm.tile[0][wave * kQRowsPerWave * kRowStride])));

  QueryState st;
  query_state_reset(st);
  for (int64_t base = s_begin; base < s_end; base += kListCap) {
    const int cnt = int(min(int64_t(kListCap), s_end - base));
    __syncthreads();  // the previous batch is done with s_list and the ring
    // ---- compaction of this batch's valid slots -----------------------------
    int vals[kSlotsPerThread];
    int c = 0;
    bool bad = false;
    int raw[kSlotsPerThread];
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i) {
      const int sl = tid * kSlotsPerThread + i;
      raw[i] = sl < cnt ? irow[base + sl] : -1;
    }
    // Q^T: issued after the index loads (which return first, so the
    // compaction waits for them alone) and complete before the first gather
    // is issued (vmcnt below). Not under a branch, so that the compiler's
    // wait for the indices counts these loads as younger; a batch after the
    // first reloads the same Q.
    query_load_q(p, bi, mi, st);
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i) {
      const int v = raw[i];
      const bool ok = (v >= 0) && (int64_t(v) < p.kv_len);
      bad |= (!ok && v != -1);
      vals[i] = ok ? v : -1;
      c += ok ? 1 : 0;
    }
    if (bad && p.err != nullptr) flag_bad_index(p.err);
    int incl = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
    if (lane == 63) s_cnt[wave] = incl;
    __syncthreads();
    int pos = incl - c;
    int nvalid = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int t = s_cnt[w];
      pos += (w < wave) ? t : 0;
      nvalid += t;
    }
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i)
      if (vals[i] >= 0) s_list[pos++] = vals[i];
    __syncthreads();
    if (nvalid == 0) continue;
    // An unsplit query walks its rows in ascending order. The queries of a
    // launch that share a batch's kv then sweep it together, so a row that
    // several of one XCD's queries name is fetched once into that XCD's L2
    // and read there by the others, instead of each fetch landing at a
    // random time. (A split query's parts run on many CUs at once, and a
    // decode batch has one query: nothing to align.) Softmax and the sums
    // do not depend on the slot order beyond the fp32 rounding of the sums.
    if (p.nsplit == 1) {
      if (nvalid <= kThreads)
        sort_list<1>(s_list, nvalid);
      else if (nvalid <= 2 * kThreads)
        sort_list<2>(s_list, nvalid);
      else if (nvalid <= 4 * kThreads)
        sort_list<4>(s_list, nvalid);
      else
        sort_list<8>(s_list, nvalid);
    }
    const int nsteps = (nvalid + kQRows - 1) / kQRows;
    // every load of this wave (Q) is complete before the gathers, whose
    // ring waits count only them
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

    // ---- gather ring -----------------------------------------------------------
    // Wave w gathers rows 8w..8w+7 of a step; lane i < 8 reads the list entry
    // of row i, and each row's address is a scalar base (readlane). Entries
    // past the last valid one take entry 0's row; their scores are masked.
    auto issue = [&](int step) {
      const int e = step * kQRows + wave * kQRowsPerWave + (lane & 7);
      const int rv = s_list[e < nvalid ? e : 0];
      const uint32_t lbase = lds_rows + uint32_t((step % kQRing) * kQRows * kRowStride);
#pragma unroll
      for (int i = 0; i < kQRowsPerWave; ++i) {
        const int row = __builtin_amdgcn_readlane(rv, i);
        lds_dma_row(kvb + int64_t(row) * row_bytes, 16 * lane, lbase + uint32_t(i * kRowStride));
      }
    };
    for (int s = 0; s < min(kQAhead, nsteps); ++s) issue(s);

    for (int step = 0; step < nsteps; ++step) {
      wait_ring(min(nsteps - 1, step + kQAhead - 1) - step);
      lds_barrier();  // every wave's rows of `step` are in LDS; the previous buffer is free
      // the list entries of the rows this wave gathers for step + kQAhead
      const int sg = step + kQAhead;
      int rv = 0;
      if (sg < nsteps) {
        const int e = sg * kQRows + wave * kQRowsPerWave + (lane & 7);
        rv = s_list[e < nvalid ? e : 0];
      }
      const uint32_t lbase = lds_rows + uint32_t((sg % kQRing) * kQRows * kRowStride);
      query_step<kRing>(p, sm, sm.tile[step % kQRing], sg < nsteps, rv, lbase, kvb, row_bytes,
                        nvalid - step * kQRows, st, [] {});
    }
  }
  query_epilogue<kRing>(p, sm, unit, bi, mi, st);
}

// The queries m0 .. m0 + nq - 1 of batch bi (nq <= kTQ, nq * topk <= kListCap,
// no split) as one stream of steps through a 2-deep ring. Their valid slots
// are compacted into the list at once (query j's at qs[j] .. qs[j + 1]), so
// a query's first gathers are issued during the previous query's last step
// and its Q^T loads once that step's S^T is done: the index loads, the
// compaction and the first gather latency are paid once per tile instead of
// once per query. The list holds the rows' 32-bit byte offsets in the
// batch's kv (a shared-row plan guarantees they fit).
// The compiler does not see the LDS-DMA gathers, so every step's ring wait
// (vmcnt(0) with 2 buffers) is also made as a builtin the compiler sees: its
// count of outstanding loads then never holds a Q^T load, and it puts no wait
// of its own between the gathers of a step.
template <int kRing>
__device__ __forceinline__ void query_stream(const FwdParams& p, int64_t bi, int64_t m0, int nq,
                                             QuerySmemT<kRing>& sm) {
  static_assert(kRing == 2, "the stream's waits are those of a 2-deep ring");
  constexpr int kQAhead = kRing - 1;
  auto& s_list = sm.list;
  auto& s_cnt = sm.cnt;
  auto& s_qs = sm.qstart;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int topk = int(p.topk);
  const int nslots = nq * topk;
  const uint8_t* kvb = reinterpret_cast<const uint8_t*>(p.kv + bi * p.skv_b);
  const int64_t row_bytes = p.skv_n * 2;
  const int32_t* ib = p.idx + bi * p.si_b + m0 * p.si_m;
  const uint32_t lds_rows = __builtin_amdgcn_readfirstlane(uint32_t(
      reinterpret_cast<uintptr_t>((lds_u8_t*)&sm.tile[0][wave * kQRowsPerWave * kRowStride])));

  // ---- compaction of the tile's valid slots, query by query -------------------
  // thread tid holds slots tid * kSlotsPerThread + i: query j0 + .., slot k0 + ..
  const int sl0 = tid * kSlotsPerThread;
  const int j0 = sl0 / topk;
  const int k0 = sl0 - j0 * topk;
  int raw[kSlotsPerThread];
  {
    int j = j0, k = k0;
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i) {
      raw[i] = sl0 + i < nslots ? ib[j * p.si_m + k] : -1;
      if (++k == topk) {
        k = 0;
        ++j;
      }
    }
  }
  QueryState st;
  query_state_reset(st);
  query_load_q(p, bi, m0, st);  // query 0's (reloaded below if it has no valid slot)
  int vals[kSlotsPerThread];
  int c = 0;
  bool bad = false;
#pragma unroll
  for (int i = 0; i < kSlotsPerThread; ++i) {
    const int v = raw[i];
    const bool ok = (v >= 0) && (int64_t(v) < p.kv_len);
    bad |= (!ok && v != -1);
    vals[i] = ok ? v : -1;
    c += ok ? 1 : 0;
  }
  if (bad && p.err != nullptr) flag_bad_index(p.err);
  int incl = c;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off);
    if (lane >= off) incl += t;
  }
  if (lane == 63) s_cnt[wave] = incl;
  __syncthreads();
  int pos = incl - c;
  int nvalid = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int t = s_cnt[w];
    pos += (w < wave) ? t : 0;
    nvalid += t;
  }
  {
    int j = j0, k = k0;
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i) {
      if (k == 0 && sl0 + i < nslots) s_qs[j] = pos;  // a query's first slot
      if (vals[i] >= 0) s_list[pos++] = int32_t(uint32_t(vals[i]) * uint32_t(row_bytes));
      if (++k == topk) {
        k = 0;
        ++j;
      }
    }
  }
  if (tid == 0) s_qs[nq] = nvalid;
  __syncthreads();
  int qs[kTQ + 1];
#pragma unroll
  for (int j = 0; j <= kTQ; ++j) qs[j] = j <= nq ? __builtin_amdgcn_readfirstlane(s_qs[j]) : nvalid;
  auto nst = [&](int j) { return (qs[j + 1] - qs[j] + kQRows - 1) / kQRows; };
  int total = 0;
#pragma unroll
  for (int j = 0; j < kTQ; ++j) total += j < nq ? nst(j) : 0;
  // Q^T (and the indices) complete before the first gather is issued
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // ---- the step stream ----------------------------------------------------------
  // The issue cursor (ji, si): query and step of the next step to gather.
  // Entries past a query's last valid one take its first entry's row; their
  // scores are masked.
  int ji = 0, si = 0;
  while (ji < nq && nst(ji) == 0) ++ji;
  auto cursor_rows = [&]() {
    const int e = qs[ji] + si * kQRows + wave * kQRowsPerWave + (lane & 7);
    const int rv = s_list[e < qs[ji + 1] ? e : qs[ji]];
    if (++si == nst(ji)) {
      si = 0;
      do {
        ++ji;
      } while (ji < nq && nst(ji) == 0);
    }
    return rv;
  };
  if (total > 0) {
    const int rv = cursor_rows();
#pragma unroll
    for (int i = 0; i < kQRowsPerWave; ++i) {
      const uint32_t off = uint32_t(__builtin_amdgcn_readlane(rv, i));
      lds_dma_row(kvb + off, 16 * lane, lds_rows + uint32_t(i * kRowStride));
    }
  }
  int gstep = 0;
  int qloaded = 0;  // the query whose Q^T is in st.qf
  for (int j = 0; j < nq; ++j) {
    const int ns = nst(j);
    int jn = j + 1;  // the next query with a valid slot
    while (jn < nq && nst(jn) == 0) ++jn;
    if (ns > 0 && qloaded != j) {  // only after a query without a valid slot
      query_load_q(p, bi, m0 + j, st);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      qloaded = j;
    }
    for (int s = 0; s < ns; ++s, ++gstep) {
      wait_ring(0);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // the same wait, for the compiler's count
      lds_barrier();  // every wave's rows of this step are in LDS; the other buffer is free
      const bool dma = gstep + kQAhead < total;
      const int rv = dma ? cursor_rows() : 0;
      const uint32_t lbase =
          lds_rows + uint32_t(((gstep + kQAhead) % kRing) * kQRows * kRowStride);
      const bool last = s == ns - 1;
      query_step<kRing, true>(p, sm, sm.tile[gstep % kRing], dma, rv, lbase, kvb, row_bytes,
                              qs[j + 1] - qs[j] - s * kQRows, st, [&] {
                                if (last && jn < nq) query_load_q(p, bi, m0 + jn, st);
                              });
    }
    if (ns > 0 && jn < nq) qloaded = jn;
    query_epilogue<kRing>(p, sm, bi * p.m + m0 + j, bi, m0 + j, st);
    query_state_reset(st);
  }
}

// ============================================================================
// tile index kernel
// ============================================================================
// Builds, for one tile of kTQ consecutive queries, the ascending union of the
// rows its valid slots name and each row's multiplicity in every query.
// Multiplicity layout of a tile: for step s (64 union entries) and tile query
// q, the 64 values of the step's rows are contiguous at ((s * kTQ) + q) * 64.
// A value is log2 of the row's count in the query as fp16 (exact for powers of
// two, within 2^-11 relative otherwise) or -inf when the query does not name
// the row, so that s * scale + value is the masked, multiplicity-weighted
// score in the log2 domain. A lane reads 4 consecutive rows of its query as
// 8 bytes.
// One work-group of kIdxThreads per tile. Three phases, each with many
// independent memory operations in flight per wave:
//  1. count: the tile's indices are read as int4 (int32 when the index rows
//     are not 16-byte aligned), kIdxVec per thread per round, all of a round
//     issued before any is used; every valid index is added to the u64 LDS
//     counter of its row (byte q = count in tile query q), and the valid
//     slots are counted with ballots.
//  2. scan: wave w takes a contiguous run of 64-row chunks and counts its
//     nonzero rows, its first row and the sum of all count bytes, reading
//     kIdxScan chunks per batch. A count passing 255 carries into the next
//     byte (or out of the word) and lowers that sum, so a sum below the
//     valid slots makes the tile per-query.
//  3. write: the waves' run lengths give each its first union entry; a
//     ballot per chunk ranks the nonzero rows, so the union is written in
//     ascending row order with consecutive lanes on consecutive entries.
// 1024 threads with 2 vectors per round from kIdxWideKv rows (the count
// table then allows one work-group per CU): the 1x16384 kv_len 16384 topk 128
// shape's index kernel 31.6 -> 26.1 us; 512 threads with 4 vectors below,
// and 256 threads for tiles of at most 4 096 slots (one round of 1 or 4
// vectors per thread, and twice the work-groups per CU): the contest shapes'
// index kernel 64x1024-1024-128 36.7 -> 13.2 us, 16x4096-4096-128 40.0 ->
// 21.3, 64x1024-1280-384 101 -> 73 (A/B, same box).
// The one-wave kernel's list holds this many slots per query (queries with
// topk up to it run one wave each). Against the 4-wave per-query kernel:
// topk 128 1365 -> 1102 us/call at 64 x 1024 queries, topk 640 1232 -> 1260
// at 1 x 16384 (a longer list amortises that kernel's start), so the cap sits
// between them.
constexpr int kWaveMaxTopk = 384;
constexpr int kIdxThreadsNarrow = 512;
constexpr int kIdxVecNarrow = 4;    // index vectors per thread per round
constexpr int64_t kIdxWideKv = 8192;
constexpr int kIdxSmallSlots = 4096;  // tile slots (8 topk) up to which 256 threads
constexpr int kIdxScan = 4;   // LDS chunk reads per wave per batch

// kBits (long caches, topk <= kWaveMaxTopk, whose tiles usually go per
// query): the tile's valid rows are first marked in a bitmap (the count
// table's first kv_len / 8 bytes), which gives the union size and so the
// mode; only a shared tile then clears the count table and counts, from the
// same index registers (one round holds the tile's indices).
template <int kIdxThreads, int kIdxVec, bool kBits>
__global__ void __launch_bounds__(kIdxThreads) sa_tile_index_kernel(const IndexParams p) {
  constexpr int kIdxWaves = kIdxThreads / 64;
  extern __shared__ unsigned long long s_count[];  // [kv_len], byte q = count in query q
  constexpr int kMaxChunks = int(sa::kMaxTileKv / 64);
  __shared__ uint8_t s_cnz[kMaxChunks];    // 64-row chunk holds a named row
  __shared__ int16_t s_clist[kMaxChunks];  // those chunks, ascending
  __shared__ int s_nchunks;
  __shared__ int s_wtot[kIdxWaves];
  __shared__ int s_nvalid;   // valid slots of the tile
  __shared__ int s_nunion;   // rows named by the tile (first counts of a row)
  __shared__ int s_bytes;    // sum of every count byte
  __shared__ int s_first;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t tile = blockIdx.x;
  const int64_t bi = tile / p.tiles_per_b;
  const int64_t q0 = (tile % p.tiles_per_b) * kTQ;
  const int qt = int(min(int64_t(kTQ), p.m - q0));
  const int kvl = int(p.kv_len);
  const int topk = int(p.topk);

  const int nchunks = (kvl + 63) / 64;
  const int32_t* ib = p.idx + bi * p.si_b + q0 * p.si_m;
  bool bad = false;  // an index outside [-1, kv_len)
  int nvalid = 0;    // wave-uniform
  int nfresh = 0;    // this lane's counts that found their row's word at 0
  auto count = [&](int v, int qq) {
    const bool ok = v >= 0 && v < kvl;
    if (ok) {
      nfresh += atomicAdd(&s_count[v], 1ull << (8 * qq)) == 0ull ? 1 : 0;
      s_cnz[v >> 6] = 1;
    }
    bad = bad || (!ok && v != -1);
    nvalid += __popcll(__ballot(ok));
  };
  // vec4: topk, the row strides and the base are multiples of 4 int32
  const int rv = topk / 4;  // int4 per query row
  const int nv4 = qt * rv;
  auto load4 = [&](int e0, int4 (&v)[kIdxVec], int (&qv)[kIdxVec]) {
#pragma unroll
    for (int u = 0; u < kIdxVec; ++u) {
      const int e = e0 + u * kIdxThreads + tid;
      const int qq = e / max(rv, 1);
      qv[u] = qq;
      v[u] = e < nv4 ? *reinterpret_cast<const int4*>(ib + qq * p.si_m + 4 * (e - qq * rv))
                     : int4{-1, -1, -1, -1};
    }
  };
  auto count4 = [&](const int4 (&v)[kIdxVec], const int (&qv)[kIdxVec]) {
#pragma unroll
    for (int u = 0; u < kIdxVec; ++u) {
      count(v[u].x, qv[u]);
      count(v[u].y, qv[u]);
      count(v[u].z, qv[u]);
      count(v[u].w, qv[u]);
    }
  };
  // The first round of index loads flies while the count table is cleared.
  int4 v0[kIdxVec];
  int q0v[kIdxVec];
  if (p.vec4) load4(0, v0, q0v);
  // kBits without vec4: the tile's indices as int32, one round
  int vs[4 * kIdxVec];
  int qs[4 * kIdxVec];
  if constexpr (kBits) {
    static_assert(kIdxThreads * kIdxVec * 4 >= kTQ * kWaveMaxTopk, "one round holds a tile");
    if (!p.vec4) {
      const int nv = qt * topk;
#pragma unroll
      for (int u = 0; u < 4 * kIdxVec; ++u) {
        const int e = u * kIdxThreads + tid;
        const int qq = e / max(topk, 1);
        qs[u] = qq;
        vs[u] = e < nv ? ib[qq * p.si_m + (e - qq * topk)] : -1;
      }
    }
    // ---- 0. mark: the union size and the mode ------------------------------------
    uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_count);
    for (int i = tid; i < (kvl + 31) / 32; i += kIdxThreads) s_bits[i] = 0u;
    if (tid == 0) {
      s_nvalid = 0;
      s_nunion = 0;
    }
    __syncthreads();
    auto mark = [&](int v) {
      const bool ok = v >= 0 && v < kvl;
      if (ok) {
        const uint32_t bit = 1u << (v & 31);
        nfresh += (atomicOr(&s_bits[v >> 5], bit) & bit) == 0u ? 1 : 0;
      }
      bad = bad || (!ok && v != -1);
      nvalid += __popcll(__ballot(ok));
    };
    if (p.vec4) {
#pragma unroll
      for (int u = 0; u < kIdxVec; ++u) {
        mark(v0[u].x);
        mark(v0[u].y);
        mark(v0[u].z);
        mark(v0[u].w);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4 * kIdxVec; ++u) mark(vs[u]);
    }
    if (bad && p.err != nullptr) flag_bad_index(p.err);
    if (lane == 0 && nvalid != 0) atomicAdd(&s_nvalid, nvalid);
    for (int off = 32; off > 0; off >>= 1) nfresh += __shfl_xor(nfresh, off);
    if (lane == 0 && nfresh != 0) atomicAdd(&s_nunion, nfresh);
    __syncthreads();
    // the first setter of each row's bit counted it: s_nunion is the union size
    const bool cheaper = shared_is_cheaper(s_nunion, s_nvalid, qt, p.placed_regime != 0);
    if (p.force == 0 && !cheaper) {
      if (tid == 0) {
        int32_t* meta = p.meta + tile * kMetaInts;
        meta[0] = s_nunion;
        meta[1] = sa::kModePerQuery;
        meta[2] = s_nvalid;
        meta[3] = 0;
      }
      return;
    }
    __syncthreads();  // every thread has read the counts; the bitmap is free
  }
  for (int i = tid; i < kvl; i += kIdxThreads) s_count[i] = 0ull;
  for (int i = tid; i < nchunks; i += kIdxThreads) s_cnz[i] = 0;
  if (tid == 0) {
    s_first = kvl;
    if (!kBits) {
      s_nvalid = 0;
      s_nunion = 0;
    }
    s_bytes = 0;
  }
  __syncthreads();

  // ---- 1. count --------------------------------------------------------------
  if constexpr (kBits) {
    // the mode is decided and the valid slots counted: the counts alone
    auto count_row = [&](int v, int qq) {
      if (v >= 0 && v < kvl) {
        atomicAdd(&s_count[v], 1ull << (8 * qq));
        s_cnz[v >> 6] = 1;
      }
    };
    if (p.vec4) {
#pragma unroll
      for (int u = 0; u < kIdxVec; ++u) {
        count_row(v0[u].x, q0v[u]);
        count_row(v0[u].y, q0v[u]);
        count_row(v0[u].z, q0v[u]);
        count_row(v0[u].w, q0v[u]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4 * kIdxVec; ++u) count_row(vs[u], qs[u]);
    }
    __syncthreads();
  } else if (p.vec4) {
    count4(v0, q0v);
    for (int e0 = kIdxThreads * kIdxVec; e0 < nv4; e0 += kIdxThreads * kIdxVec) {
      int4 v[kIdxVec];
      int qv[kIdxVec];
      load4(e0, v, qv);
      count4(v, qv);
    }
  } else {
    const int nv = qt * topk;
    for (int e0 = 0; e0 < nv; e0 += kIdxThreads * kIdxVec * 4) {
      int v[4 * kIdxVec];
      int qv[4 * kIdxVec];
#pragma unroll
      for (int u = 0; u < 4 * kIdxVec; ++u) {
        const int e = e0 + u * kIdxThreads + tid;
        const int qq = e / max(topk, 1);
        qv[u] = qq;
        v[u] = e < nv ? ib[qq * p.si_m + (e - qq * topk)] : -1;
      }
#pragma unroll
      for (int u = 0; u < 4 * kIdxVec; ++u) count(v[u], qv[u]);
    }
  }
  if constexpr (!kBits) {
    if (bad && p.err != nullptr) flag_bad_index(p.err);
    if (lane == 0 && nvalid != 0) atomicAdd(&s_nvalid, nvalid);
    for (int off = 32; off > 0; off >>= 1) nfresh += __shfl_xor(nfresh, off);
    if (lane == 0 && nfresh != 0) atomicAdd(&s_nunion, nfresh);
    __syncthreads();
    // Each row's first count found its word at 0 (LDS atomics on one word
    // are serialised), so s_nunion is the union size, and the mode can be
    // decided now: a per-query tile needs no union, so its scan and write are
    // skipped. (A count carry can only make a tile per query, below.)
    const bool cheaper = shared_is_cheaper(s_nunion, s_nvalid, qt, p.placed_regime != 0);
    if (p.force == 0 && !cheaper) {
      if (tid == 0) {
        int32_t* meta = p.meta + tile * kMetaInts;
        meta[0] = s_nunion;
        meta[1] = sa::kModePerQuery;
        meta[2] = s_nvalid;
        meta[3] = 0;
      }
      return;
    }
  }

  // ---- 2. scan -----------------------------------------------------------------
  // Only the 64-row chunks holding a named row are scanned (a high-locality
  // tile names a few dozen of 256): wave 0 lists them in ascending order, and
  // wave w takes the w-th contiguous eighth of that list, so the union stays
  // in ascending row order across the waves.
  if (wave == 0) {
    int base = 0;
    for (int c0 = 0; c0 < nchunks; c0 += 64) {
      const bool nz = c0 + lane < nchunks && s_cnz[c0 + lane] != 0;
      const unsigned long long bm = __ballot(nz);
      if (nz) s_clist[base + __popcll(bm & ((1ull << lane) - 1ull))] = int16_t(c0 + lane);
      base += __popcll(bm);
    }
    if (lane == 0) s_nchunks = base;
  }
  __syncthreads();
  const int nlist = s_nchunks;
  const int cpw = (nlist + kIdxWaves - 1) / kIdxWaves;
  const int c_lo = min(nlist, wave * cpw);
  const int c_hi = min(nlist, c_lo + cpw);
  int wcount = 0;  // wave-uniform
  int wfirst = kvl;
  int bytes = 0;   // this lane's sum of count bytes
  for (int c0 = c_lo; c0 < c_hi; c0 += kIdxScan) {
    unsigned long long wv[kIdxScan];
    int ch[kIdxScan];
#pragma unroll
    for (int u = 0; u < kIdxScan; ++u) {
      ch[u] = c0 + u < c_hi ? int(s_clist[c0 + u]) : 0;
      const int i = ch[u] * 64 + lane;
      wv[u] = (c0 + u < c_hi && i < kvl) ? s_count[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < kIdxScan; ++u) {
      const unsigned long long bm = __ballot(wv[u] != 0ull);
      if (bm != 0ull && wfirst == kvl) wfirst = ch[u] * 64 + __ffsll((long long)bm) - 1;
      wcount += __popcll(bm);
      // the 8 bytes as four 16-bit pair sums, then their total
      const unsigned long long pairs =
          (wv[u] & 0x00FF00FF00FF00FFull) + ((wv[u] >> 8) & 0x00FF00FF00FF00FFull);
      bytes += int((pairs * 0x0001000100010001ull) >> 48);
    }
  }
  if (lane == 0) s_wtot[wave] = wcount;
  for (int off = 32; off > 0; off >>= 1) bytes += __shfl_xor(bytes, off);
  if (lane == 0 && bytes != 0) atomicAdd(&s_bytes, bytes);
  if (lane == 0 && wfirst < kvl) atomicMin(&s_first, wfirst);
  __syncthreads();

  // ---- 3. write ------------------------------------------------------------------
  int pos = 0;
  int nU = 0;
  for (int w = 0; w < kIdxWaves; ++w) {
    const int t = s_wtot[w];
    pos += (w < wave) ? t : 0;
    nU += t;
  }
  uint32_t* row_off = p.row_off + tile * p.cap;
  _Float16* lcnt = p.lcnt + tile * p.cap * kTQ;
  const uint32_t row_bytes = uint32_t(p.skv_n) * 2u;  // the plan keeps offsets in 32 bits
  auto put = [&](int e, int row, unsigned long long w) {
    row_off[e] = uint32_t(row) * row_bytes;
    _Float16* cb = lcnt + (e / kTileRows) * (kTQ * kTileRows) + (e % kTileRows);
#pragma unroll
    for (int k = 0; k < kTQ; ++k) {
      const unsigned c = unsigned((w >> (8 * k)) & 255ull);
      // v_log_f32 is log2; its error on 2..255 is far below fp16's half ulp
      // at the rounding (exact at powers of two after it)
      cb[k * kTileRows] = c == 0u   ? static_cast<_Float16>(-INFINITY)
                          : c == 1u ? static_cast<_Float16>(0.f)
                                    : static_cast<_Float16>(__builtin_amdgcn_logf(float(c)));
    }
  };
  const unsigned long long below = (1ull << lane) - 1ull;  // lanes under this one
  for (int c0 = c_lo; c0 < c_hi; c0 += kIdxScan) {
    unsigned long long wv[kIdxScan];
    int ch[kIdxScan];
#pragma unroll
    for (int u = 0; u < kIdxScan; ++u) {
      ch[u] = c0 + u < c_hi ? int(s_clist[c0 + u]) : 0;
      const int i = ch[u] * 64 + lane;
      wv[u] = (c0 + u < c_hi && i < kvl) ? s_count[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < kIdxScan; ++u) {
      const unsigned long long bm = __ballot(wv[u] != 0ull);
      if (wv[u] != 0ull) put(pos + __popcll(bm & below), ch[u] * 64 + lane, wv[u]);
      pos += __popcll(bm);
    }
  }
  // pad to whole 64-row steps with a valid row of count 0
  const int padded = (nU + kTileRows - 1) / kTileRows * kTileRows;
  for (int e = nU + tid; e < padded; e += kIdxThreads) put(e, s_first, 0ull);
  if (tid == 0) {
    const int total = s_nvalid;
    const bool overflow = s_bytes != total;  // a count carried
    const bool shared = !overflow;  // and cheaper, or forced (above)
    int32_t* meta = p.meta + tile * kMetaInts;
    meta[0] = nU;
    meta[1] = shared ? kModeShared : sa::kModePerQuery;
    meta[2] = total;
    meta[3] = overflow ? 1 : 0;
  }
}

// ============================================================================
// tile order (the first work-group of the per-query launch)
// ============================================================================
// One work-group sorts the tiles by descending step count (a counting sort:
// a shared tile's key is 1 + its step count, a per-query tile's 0). The
// shared-row kernel's work-group i runs entry i; work-groups start in index
// order, so the longest tiles start first and the short ones fill in at the
// end. Tiles with equal keys may come in any order: each tile is independent.
// The per-query tiles' entries come last; the shared-row kernel's
// work-groups of those entries return at once (the per-query launch runs
// their queries).
// When the shared tiles fit the first wave of the shared-row kernel's grid
// (at most one per CU, so every one starts at once) their order cannot
// change when they finish; they are then placed for L2 reuse instead. Work-
// group i runs on XCD i % 8, and XCD x gets the x-th eighth of the shared
// tiles in tile order: consecutive queries of one batch, whose row unions
// overlap and which sweep their ascending unions in step, share that XCD's L2.
constexpr int kOrderKeys = int(sa::kMaxTileKv / kTileRows) + 2;
constexpr int kOrderKeysPadded = (kOrderKeys + 63) / 64 * 64;
constexpr int kOrderPer = 8;  // tiles per thread per pass (their loads issued together)
// XCD placement handles at most this many tiles (every shared tile then
// starts at once anyway)
constexpr int kOrderPlaceMax = 1024;
// tiles whose keys the first pass keeps in LDS for the second (16-bit keys)
constexpr int kOrderKeyCache = 16384;
// With the keys cached, the 64-tile chunks whose per-query tiles are
// counted for the second pass.
constexpr int kOrderChunks = kOrderKeyCache / 64;
// threads of the order's own launch (sa_order_kernel)
constexpr int kOrderThreads = 1024;
static_assert(kOrderKeys <= (1 << (31 - kOrderTileBits)), "keys fit the order entry");

constexpr int kXcds = 8;  // MI355X: work-groups are dealt to the 8 XCDs round-robin

struct OrderSmem {
  int pos[kOrderKeysPadded];
  int wcount[kOrderThreads / 64];
  int zpre[kOrderChunks];  // per-query tiles in the 64-tile chunks before chunk c
  uint16_t key[kOrderKeyCache];
};

// Exclusive scan of n ints in LDS by one wave, in place; returns the total.
__device__ __forceinline__ int wave_exclusive_scan(int* v, int n) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  for (int c0 = 0; c0 < n; c0 += 64) {
    const int i = c0 + lane;
    const int x = i < n ? v[i] : 0;
    int incl = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
    if (i < n) v[i] = carry + incl - x;
    carry += __shfl(incl, 63);
  }
  return carry;
}

// The tile order, made by one work-group of NT threads: work-group 0 of the
// tile-plan per-query launch (NT = kThreads), or sa_order_kernel (NT =
// kOrderThreads) where that launch would do nothing else.
//  * Pass 1 reads every tile's key and counts the keys in LDS. With at most
//    kOrderKeyCache tiles, the (union size, mode) pairs of kOrderLoad tiles
//    per thread are loaded as 8-byte words, all issued before any is used,
//    and the keys stay in LDS for pass 2.
//  * The counts are scanned in descending key order.
//  * Pass 2 writes each shared tile at the next free slot of its key (an LDS
//    atomic), and each per-query tile at nshared + its rank among the
//    per-query tiles in tile order, from per-chunk counts (no atomic, so no
//    chain of atomic, shuffle and store per wave).
template <int NT>
__device__ void make_order(const OrderParams& p, OrderSmem& sm) {
  static_assert(NT % 64 == 0 && NT / 64 <= kOrderThreads / 64, "wave counts fit wcount");
  // with the keys cached: tiles per thread whose metadata loads are issued
  // together (one round covers NT * kOrderLoad tiles)
  constexpr int kOrderLoad = NT >= 1024 ? 8 : 16;
  static_assert(kOrderKeyCache % (NT * kOrderLoad) == 0, "whole load rounds");
  constexpr int kW = NT / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const unsigned long long below = (1ull << lane) - 1ull;
  const int32_t* meta = p.meta;
  const int ntiles = p.ntiles;
  for (int i = tid; i < kOrderKeysPadded; i += NT) sm.pos[i] = 0;
  __syncthreads();
  auto key_of = [](int nU, int mode) {
    return mode == kModeShared ? (nU + kTileRows - 1) / kTileRows + 1 : 0;
  };
  auto key = [&](int t) {
    const int32_t* mt = meta + int64_t(t) * kMetaInts;
    return key_of(mt[0], mt[1]);
  };
  const bool cached = ntiles <= kOrderKeyCache;
  auto keys = [&](int t0, int (&k)[kOrderPer], bool from_lds) {
#pragma unroll
    for (int u = 0; u < kOrderPer; ++u) {
      const int t = t0 + u * NT + tid;
      k[u] = t >= ntiles ? -1 : from_lds ? int(sm.key[t]) : key(t);
    }
  };
  if (cached) {
    for (int t0 = 0; t0 < ntiles; t0 += NT * kOrderLoad) {
      int2 mv[kOrderLoad];
#pragma unroll
      for (int u = 0; u < kOrderLoad; ++u) {  // clamped, so that every load is issued
        const int t = min(t0 + u * NT + tid, ntiles - 1);
        mv[u] = *reinterpret_cast<const int2*>(meta + int64_t(t) * kMetaInts);
      }
#pragma unroll
      for (int u = 0; u < kOrderLoad; ++u) {
        if (t0 + u * NT >= ntiles) break;  // (uniform) the rest of the round is past the end
        const int t = t0 + u * NT + tid;
        const int k = t >= ntiles ? -1 : key_of(mv[u].x, mv[u].y);
        const unsigned long long z = __ballot(k == 0);
        if (k > 0) atomicAdd(&sm.pos[k], 1);
        if (lane == 0 && t - lane < ntiles) sm.zpre[(t - lane) / 64] = __popcll(z);
        if (lane == 0 && z != 0ull) atomicAdd(&sm.pos[0], __popcll(z));
        if (k >= 0) sm.key[t] = uint16_t(k);
      }
    }
  } else {
    // Key 0 (every per-query tile) is counted per wave: one LDS atomic per
    // wave instead of one per tile on a single word.
    for (int t0 = 0; t0 < ntiles; t0 += NT * kOrderPer) {
      int k[kOrderPer];
      keys(t0, k, false);
#pragma unroll
      for (int u = 0; u < kOrderPer; ++u) {
        const unsigned long long z = __ballot(k[u] == 0);
        if (k[u] > 0) atomicAdd(&sm.pos[k[u]], 1);
        if (lane == 0 && z != 0ull) atomicAdd(&sm.pos[0], __popcll(z));
      }
    }
  }
  __syncthreads();
  const int nshared = ntiles - sm.pos[0];  // shared tiles: every key above 0
  __syncthreads();  // every thread has read pos[0] before the scan rewrites it
  static_assert(kOrderPlaceMax <= NT * kOrderPer && kOrderPlaceMax <= kOrderKeyCache &&
                    kOrderPlaceMax % NT == 0,
                "placement reads one pass of cached keys");
  if (nshared <= p.cus && ntiles <= kOrderPlaceMax) {
    // Every shared tile starts at once: XCD-local placement (see above). A
    // tile's rank among the shared tiles in tile order picks its slot; the
    // per-query tiles' entries fill the slots after them.
    int k[kOrderPer];
    keys(0, k, true);
    int carry = 0;  // shared tiles of the earlier blocks of NT tiles
#pragma unroll
    for (int u = 0; u < kOrderPlaceMax / NT; ++u) {
      const int t = u * NT + tid;
      const bool sh = k[u] > 0;
      const unsigned long long bm = __ballot(sh);
      if (lane == 0) sm.wcount[wave] = __popcll(bm);
      __syncthreads();
      int rank = carry + __popcll(bm & below);
      for (int w = 0; w < kW; ++w) {
        const int c = sm.wcount[w];
        rank += w < wave ? c : 0;
        carry += c;
      }
      if (t < ntiles) {
        int slot = nshared + (t - rank);  // a per-query tile: after the shared ones
        if (sh) {
          // XCD x holds the slots s < nshared with s % 8 == x: c_x of them
          int first = 0, x = 0;
          for (; x < kXcds - 1; ++x) {
            const int c = (nshared - x + kXcds - 1) / kXcds;
            if (rank < first + c) break;
            first += c;
          }
          slot = kXcds * (rank - first) + x;
        }
        p.order[slot] = ((sh ? k[u] : 0) << kOrderTileBits) | t;
      }
      __syncthreads();  // wcount is rewritten by the next block
    }
    return;
  }
  if (wave == 0) {
    // exclusive scan over descending keys: the start of key k is the number
    // of tiles with a larger key
    int carry = 0;
    for (int c = kOrderKeysPadded / 64 - 1; c >= 0; --c) {
      const int k = 64 * c + 63 - lane;  // lane 0 takes the largest key of the chunk
      const int v = sm.pos[k];
      int incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off);
        if (lane >= off) incl += t;
      }
      sm.pos[k] = carry + incl - v;
      carry += __shfl(incl, 63);
    }
  } else if (wave == 1 && cached) {
    wave_exclusive_scan(sm.zpre, (ntiles + 63) / 64);
  }
  __syncthreads();
  if (cached) {
    for (int t0 = 0; t0 < ntiles; t0 += NT * kOrderPer) {
#pragma unroll
      for (int u = 0; u < kOrderPer; ++u) {
        if (t0 + u * NT >= ntiles) break;  // (uniform)
        const int t = t0 + u * NT + tid;
        const int k = t >= ntiles ? -1 : int(sm.key[t]);
        const unsigned long long z = __ballot(k == 0);
        if (k > 0)
          p.order[atomicAdd(&sm.pos[k], 1)] = (k << kOrderTileBits) | t;
        else if (k == 0)
          p.order[nshared + sm.zpre[(t - lane) / 64] + __popcll(z & below)] = t;
      }
    }
    return;
  }
  for (int t0 = 0; t0 < ntiles; t0 += NT * kOrderPer) {
    int k[kOrderPer];
    keys(t0, k, false);
#pragma unroll
    for (int u = 0; u < kOrderPer; ++u) {
      const int t = t0 + u * NT + tid;
      const unsigned long long z = __ballot(k[u] == 0);
      int base = 0;
      if (lane == 0 && z != 0ull) base = atomicAdd(&sm.pos[0], __popcll(z));
      base = __shfl(base, 0);
      if (k[u] > 0)
        p.order[atomicAdd(&sm.pos[k[u]], 1)] = (k[u] << kOrderTileBits) | t;
      else if (k[u] == 0)
        p.order[base + __popcll(z & below)] = t;
    }
  }
}

// ============================================================================
// per-query launch
// ============================================================================
// Work-group i runs unit i (query i / nsplit, part i % nsplit). In a
// shared-row plan (FwdParams::meta set) it runs the queries of one tile in
// turn if the index kernel made that tile per query, and returns at once
// otherwise; when the call makes the tile order (FwdParams::ord.order set),
// work-group 0 makes it and tile i goes to work-group i + 1. (A per-query
// tile's queries in one work-group take about the CU time the mode rule
// charges them; short-lived work-groups, one per tile, balance better than
// fewer that stride over many queries.)
template <int kRing>
union QueryLaunchSmem {
  QuerySmemT<kRing> q;
  OrderSmem o;
};
static_assert(sizeof(OrderSmem) <= sizeof(QuerySmemT<2>), "the order adds no LDS");

// kTiles: the launch of a shared-row plan (FwdParams::meta set); else one
// unit per work-group (a separate instantiation: the tile-plan loop would
// cost the plain one scalar-register spills).
template <int kRing, bool kTiles>
__global__ void __launch_bounds__(kThreads, kRing == 2 ? 2 : 1)
    sa_fwd_query_kernel(const FwdParams p) {
  __shared__ __attribute__((aligned(16))) QueryLaunchSmem<kRing> sm;
  if constexpr (!kTiles) {
    query_unit<kRing>(p, blockIdx.x, sm.q);
  } else {
    int64_t t = blockIdx.x;
    if (p.ord.order != nullptr) {
      if (t == 0) {
        make_order<kThreads>(p.ord, sm.o);
        return;
      }
      --t;
    }
    if (__builtin_amdgcn_readfirstlane(p.meta[t * kMetaInts + 1]) == kModeShared) return;
    const int64_t m0 = (t % p.tiles_per_b) * kTQ;
    const int64_t qbase = (t / p.tiles_per_b) * p.m + m0;
    const int nq = int(min(int64_t(kTQ), p.m - m0));
    if constexpr (kRing == 2) {
      if (int64_t(nq) * p.topk <= kListCap) {
        query_stream<kRing>(p, t / p.tiles_per_b, m0, nq, sm.q);
        return;
      }
    }
    for (int j = 0; j < nq; ++j) {
      query_unit<kRing>(p, qbase + j, sm.q);
      __syncthreads();  // every wave is done with the LDS before the next query
    }
  }
}

// The tile order as a launch of its own: one work-group of kOrderThreads
// threads, where the per-query launch would only make the order (the short
// queries of a tile plan run in sa_fwd_wave_kernel, and an index plan). A
// quarter of the work per wave against the per-query launch's work-group 0:
// at 8 192 tiles the order takes 7.2 us here, 14.3 there (21.8 before its
// metadata loads were issued together and its per-query slots were counted
// per chunk).
__global__ void __launch_bounds__(kOrderThreads) sa_order_kernel(const OrderParams p) {
  __shared__ __attribute__((aligned(16))) OrderSmem sm;
  make_order<kOrderThreads>(p, sm);
}

// ============================================================================
// per-query wave launch
// ============================================================================
// For short queries (topk <= kWaveMaxTopk, no split): one wave64 work-group
// per kWQueries consecutive queries (of a per-query tile in a shared-row
// plan, else of the flattened b x m), run as
// one stream of kWRows-row steps through the wave's own 2-deep LDS ring, with
// no barrier and no exchange with another wave. Per step:
//  * S^T = K . Q^T with v_mfma_f32_16x16x32_bf16 (16 rows x 16 heads, K = d,
//    Q^T resident in registers); the 16 gathers of the next step ride between
//    its 16 MFMAs;
//  * the online softmax of the 16 heads inside the wave (a head's 16 scores
//    sit in 4 lanes x 4 values);
//  * O += P . V with v_mfma_f32_16x16x16_bf16. The S^T accumulator layout
//    (lane (head n, g) holds rows 4g..4g+3) is that MFMA's A operand layout,
//    so P stays in registers; V comes from the same LDS rows by transposing
//    reads.
// Four work-groups fit in a CU's LDS, one per SIMD, and a CU takes the next
// one as soon as one ends, so one wave's start and end overlap the others'
// steps. The list holds 32-bit byte offsets of the rows in the query's batch
// of kv (the host checks that they fit).
constexpr int kWRows = 16;               // rows per step
constexpr int kWPitch = kRowBytes + 48;  // LDS row pitch (bytes)
constexpr int kWQueries = 2;             // queries per work-group
constexpr int kWVAhead = 8;              // V fragments in flight in O += P . V
// A batch's kv span (bytes) above which the wave kernel sorts each query's
// rows: an XCD's L2 (4 MiB on MI355X)
constexpr int64_t kWaveSortBytes = int64_t(4) << 20;
constexpr int kWSlots = kWaveMaxTopk / 64;
static_assert(kTQ % kWQueries == 0, "a tile's queries split evenly");
static_assert(kWQueries == 2, "the cursor state is two queries' scalars");
static_assert(kDim / 32 == kWRows, "one gather per S^T MFMA");

struct WaveSmem {
  uint8_t tile[2][kWRows * kWPitch];
  int32_t list[kWQueries * kWaveMaxTopk];
};
static_assert(4 * sizeof(WaveSmem) <= 160 * 1024, "four work-groups per CU");

// Stores query (bi, mi)'s o (and lse) from the wave's state: lane (n, g)
// holds O[head 4g + j][16 blk + n]. Lanes n and n ^ 1 swap half their values
// (DPP), so that each store writes two adjacent columns of one head: the even
// lane heads 4g and 4g + 1, the odd lane heads 4g + 2 and 4g + 3. Needs o and
// its strides 4-byte aligned (validate() asks for 16 bytes).
__device__ __forceinline__ void wave_epilogue(const FwdParams& p, int64_t bi, int64_t mi,
                                              float m_run, float l_run, const f32x4 (&oacc)[32]) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  const float lt = wave_sum16(l_run);
  float lse;
  const float f = sink_fold(m_run, lt, p.sink[n] * kLog2e, lse);
  if (p.lse != nullptr && g == 0) p.lse[bi * p.sl_b + mi * p.sl_m + int64_t(n) * p.sl_h] = lse;
  float fj[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) fj[j] = __shfl(f, 4 * g + j);
  const bool odd = (n & 1) != 0;
  __bf16* const r0 =
      p.o + bi * p.so_b + mi * p.so_m + int64_t(4 * g + (odd ? 2 : 0)) * p.so_h + (n & ~1);
  __bf16* const r1 = r0 + p.so_h;
  auto swap = [](float x) {  // the value of lane n ^ 1
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
  };
#pragma unroll
  for (int blk = 0; blk < 32; ++blk) {
    const float v0 = oacc[blk][0] * fj[0], v1 = oacc[blk][1] * fj[1];
    const float v2 = oacc[blk][2] * fj[2], v3 = oacc[blk][3] * fj[3];
    const float x0 = swap(odd ? v0 : v2);
    const float x1 = swap(odd ? v1 : v3);
    const f32x2 a = odd ? f32x2{x0, v2} : f32x2{v0, x0};
    const f32x2 b = odd ? f32x2{x1, v3} : f32x2{v1, x1};
    const bf16x2 ha = __builtin_convertvector(a, bf16x2);
    const bf16x2 hb = __builtin_convertvector(b, bf16x2);
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, ha),
                                reinterpret_cast<uint32_t*>(r0 + 16 * blk));
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, hb),
                                reinterpret_cast<uint32_t*>(r1 + 16 * blk));
  }
}

// In a shared-row plan (FwdParams::meta set) work-group i runs queries
// kWQueries * (i % parts) .. of tile i / parts (parts = kTQ / kWQueries) when
// the index kernel made that tile per query; else queries kWQueries * i .. of
// the p.nblocks queries of b x m (two of them may be in different batches).
__global__ void __launch_bounds__(64, 1) sa_fwd_wave_kernel(const FwdParams p) {
  __shared__ __attribute__((aligned(16))) WaveSmem sm;
  constexpr int kParts = kTQ / kWQueries;
  const int lane = threadIdx.x;
  const int n = lane & 15;
  const int g = lane >> 4;
  int64_t q0;  // the first query, as b * m + m
  int nq;
  if (p.meta != nullptr) {
    const int64_t t = blockIdx.x / kParts;
    const int64_t m0 = (t % p.tiles_per_b) * kTQ + (blockIdx.x % kParts) * kWQueries;
    if (__builtin_amdgcn_readfirstlane(p.meta[t * kMetaInts + 1]) == kModeShared) return;
    nq = int(min(int64_t(kWQueries), p.m - m0));
    q0 = (t / p.tiles_per_b) * p.m + m0;
  } else {
    q0 = int64_t(blockIdx.x) * kWQueries;
    nq = int(min(int64_t(kWQueries), p.nblocks - q0));
  }
  if (nq <= 0) return;
  // batch and query of the two queries, as scalars (small arrays indexed by a
  // loop variable end up in LDS, and what is read from there is not known
  // to be uniform)
  const int64_t qb0 = q0 / p.m, qm0 = q0 - qb0 * p.m;
  const int64_t q1 = q0 + (nq > 1 ? 1 : 0);
  const int64_t qb1 = q1 / p.m, qm1 = q1 - qb1 * p.m;
  auto qb_of = [&](int j) { return j == 0 ? qb0 : qb1; };
  auto qm_of = [&](int j) { return j == 0 ? qm0 : qm1; };
  auto kv_of = [&](int j) {
    return reinterpret_cast<const uint8_t*>(p.kv + qb_of(j) * p.skv_b);
  };
  const int topk = int(p.topk);
  const uint32_t row_bytes = uint32_t(p.skv_n * 2);

  // ---- indices, then query 0's Q^T (B operand: lane (n, g) holds head n,
  // d = 32s + 8g .. +7 for k-step s) ----------------------------------------------
  int raw[kWQueries][kWSlots];
#pragma unroll
  for (int j = 0; j < kWQueries; ++j)
#pragma unroll
    for (int i = 0; i < kWSlots; ++i) {
      const int sl = 64 * i + lane;
      raw[j][i] = (j < nq && sl < topk) ? p.idx[qb_of(j) * p.si_b + qm_of(j) * p.si_m + sl] : -1;
    }
  bf16x8 qf[kDim / 32];
  auto load_q = [&](int j) {
    const __bf16* qrow =
        p.q + qb_of(j) * p.sq_b + qm_of(j) * p.sq_m + int64_t(n) * p.sq_h + 8 * g;
#pragma unroll
    for (int s = 0; s < kDim / 32; ++s) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
  };
  // Q^T as the B operand of S^T lives in AGPRs: qa is written from qf once
  // per query (the tied asm operand makes the compiler copy qf into the
  // AGPRs there), and the MFMAs read it with an "a" constraint. Read straight
  // from qf, the MFMAs made the compiler copy Q^T into AGPRs at every step
  // (64 v_accvgpr_write per step), since qf changes inside the step loop when
  // the next query's Q^T is loaded.
  bf16x8 qa[kDim / 32];
  auto q_to_agpr = [&]() {
#pragma unroll
    for (int s = 0; s < kDim / 32; ++s) asm volatile("" : "=a"(qa[s]) : "0"(qf[s]));
  };
  load_q(0);

  // ---- compaction: query j's valid slots at list[qsel(j) .. qsel(j + 1)) ----------
  const unsigned long long below = (1ull << lane) - 1ull;
  int pos = 0, qs1 = 0;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < kWQueries; ++j) {
    if (j == 1) qs1 = pos;
#pragma unroll
    for (int i = 0; i < kWSlots; ++i) {
      const int v = raw[j][i];
      const bool ok = (v >= 0) && (int64_t(v) < p.kv_len);
      bad |= (!ok && v != -1);
      const unsigned long long bm = __ballot(ok);
      if (ok) sm.list[pos + __popcll(bm & below)] = int32_t(uint32_t(v) * row_bytes);
      pos += __popcll(bm);
    }
  }
  const int qs2 = pos;
  if (bad && p.err != nullptr) flag_bad_index(p.err);
  __syncthreads();  // the list is written before it is read
  auto qsel = [&](int j) { return j <= 0 ? 0 : j == 1 ? qs1 : qs2; };
  auto nst = [&](int j) { return (qsel(j + 1) - qsel(j) + kWRows - 1) / kWRows; };
  int total = 0;
#pragma unroll
  for (int j = 0; j < kWQueries; ++j) total += nst(j);
  // Q^T and the indices complete before the first gather is issued, so that
  // every later vmcnt(0) waits for the ring (and a Q^T issued after a gather)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  if (p.sort_wave) {
    // Each query walks its rows in ascending order: the queries resident on
    // an XCD then sweep their batch's kv together, and a row that several of
    // them name is fetched into the XCD's L2 once. The sorted sequence does
    // not depend on the input order.
    auto sort_query = [&](int j) {
      uint32_t* s = reinterpret_cast<uint32_t*>(&sm.list[qsel(j)]);
      const int n = qsel(j + 1) - qsel(j);
      if (n <= 64)
        sort_list_wave<1>(s, n);
      else if (n <= 128)
        sort_list_wave<2>(s, n);
      else if (n <= 256)
        sort_list_wave<4>(s, n);
      else
        sort_list_wave<8>(s, n);
    };
    static_assert(kWaveMaxTopk <= 64 * 8, "the sort covers a query's slots");
    sort_query(0);
    if (nq > 1) sort_query(1);
  }

  // ---- the step stream ------------------------------------------------------------
  // The issue cursor (ji, si): query and step of the next step to gather. Lane
  // n < 16 holds the entry of the step's row n; entries past a query's last
  // valid one take its first entry's row, whose scores are masked.
  const uint32_t lds_rows = __builtin_amdgcn_readfirstlane(
      uint32_t(reinterpret_cast<uintptr_t>((lds_u8_t*)&sm.tile[0][0])));
  int ji = 0, si = 0;
  while (ji < kWQueries && nst(ji) == 0) ++ji;
  // the rows' entries for the cursor's step; kvg = the base of their batch
  const uint8_t* kvg = nullptr;
  auto cursor_rows = [&]() {
    const int e0 = qsel(ji);
    const int e = e0 + si * kWRows + n;
    const int rv = sm.list[e < qsel(ji + 1) ? e : e0];
    kvg = kv_of(ji);
    if (++si == nst(ji)) {
      si = 0;
      do {
        ++ji;
      } while (ji < kWQueries && nst(ji) == 0);
    }
    return rv;
  };
  // kvg as a scalar (for the gathers' scalar base). readfirstlane returns
  // int: each half goes through uint32_t so the low one is not sign-extended.
  auto kv_scalar = [&]() {
    const uint64_t a = reinterpret_cast<uint64_t>(kvg);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a))));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32))));
    return reinterpret_cast<const uint8_t*>(uint64_t(lo) | uint64_t(hi) << 32);
  };
  if (total > 0) {
    const int rv = cursor_rows();
    const uint8_t* kvs = kv_scalar();
#pragma unroll
    for (int i = 0; i < kWRows; ++i) {
      const uint32_t off = uint32_t(__builtin_amdgcn_readlane(rv, i));
      lds_dma_row(kvs + off, 16 * lane, lds_rows + uint32_t(i * kWPitch));
    }
  }

  f32x4 oacc[32];
  float m_run = -INFINITY, l_run = 0.f;
#pragma unroll
  for (int blk = 0; blk < 32; ++blk) oacc[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
  int gstep = 0;
  int qloaded = 0;  // the query whose Q^T is in qf
  for (int j = 0; j < nq; ++j) {
    const int ns = nst(j);
    int jn = j + 1;  // the next query with a valid slot
    while (jn < nq && nst(jn) == 0) ++jn;
    if (ns > 0 && qloaded != j) {  // only after a query without a valid slot
      load_q(j);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      qloaded = j;
    }
    for (int s = 0; s < ns; ++s, ++gstep) {
      // this step's rows (and a Q^T issued during the last step) have landed,
      // and the reads of the buffer the next gathers fill are complete
      __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
      asm volatile("" ::: "memory");
      if (s == 0) q_to_agpr();  // this query's Q^T, landed
      const bool dma = gstep + 1 < total;
      const int rv = dma ? cursor_rows() : 0;
      const uint8_t* kvs = kv_scalar();
      const uint32_t lnext = lds_rows + uint32_t(((gstep + 1) & 1) * kWRows * kWPitch);
      const uint8_t* tb = sm.tile[gstep & 1];
      const int nrows = qsel(j + 1) - qsel(j) - s * kWRows;

      // S^T for the step's 16 rows (A: lane (row n, g) reads d = 32s + 8g ..);
      // two accumulator chains, K fragments read 3 MFMAs ahead
      f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
      const uint8_t* krow = tb + n * kWPitch + 16 * g;
      auto s_chain = [&](auto with_dma) {
        bf16x8 kf[4];
#pragma unroll
        for (int k = 0; k < 3; ++k) kf[k] = *reinterpret_cast<const bf16x8*>(krow + 64 * k);
#pragma unroll
        for (int k = 0; k < kDim / 32; ++k) {
          if (k + 3 < kDim / 32)
            kf[(k + 3) & 3] = *reinterpret_cast<const bf16x8*>(krow + 64 * (k + 3));
          if (k & 1)
            mfma32_bagpr(sb, kf[k & 3], qa[k]);
          else
            mfma32_bagpr(sa, kf[k & 3], qa[k]);
          if constexpr (decltype(with_dma)::value) {
            const uint32_t off = uint32_t(__builtin_amdgcn_readlane(rv, k));
            lds_dma_row(kvs + off, 16 * lane, lnext + uint32_t(k * kWPitch));
          }
          __builtin_amdgcn_sched_barrier(0);  // keep the interleave
        }
      };
      if (dma)
        s_chain(std::true_type{});
      else
        s_chain(std::false_type{});
      // The first V fragments of O += P . V (they do not depend on P) are
      // read now, so that their LDS latency passes under the softmax: lane
      // (n, g) reads V[rows 4g .. 4g + 3][16 blk + n] of column block blk.
      const uint8_t* vb = tb + (4 * g + (n >> 2)) * kWPitch + 8 * (n & 3);
      bf16x4 vf[kWVAhead];
#pragma unroll
      for (int i = 0; i < kWVAhead; ++i) vf[i] = lds_read_tr16(vb + 32 * i);
      mfma_agpr_drain();  // S^T is read by VALU below
      if (s == ns - 1 && jn < nq) load_q(jn);  // Q^T is no longer read

      // online softmax: lane (n, g) holds S[head n][row 4g + j]
      float sv[4];
      float mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        sv[k] = (4 * g + k < nrows) ? (sa[k] + sb[k]) * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, sv[k]);
      }
      mx = wave_max16(mx);  // finite: the step's row 0 is valid
      float alpha = 1.f;
      if (mx > m_run + kRescaleLog2) {
        // (O, l still 0 at first; v_exp_f32 as in the per-query step)
        alpha = m_run == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - mx);
        m_run = mx;
      }
      float psum = 0.f;
      bf16x4 pb;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float pk = __builtin_amdgcn_exp2f(sv[k] - m_run);
        psum += pk;
        pb[k] = static_cast<__bf16>(pk);
      }
      l_run = l_run * alpha + psum;
      if (__any(alpha != 1.f)) {
        float ak[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) ak[k] = __shfl(alpha, 4 * g + k);
#pragma unroll
        for (int blk = 0; blk < 32; ++blk)
#pragma unroll
          for (int k = 0; k < 4; ++k) oacc[blk][k] *= ak[k];
      }

      // O += P . V over the 32 column blocks, each V fragment read kWVAhead
      // MFMAs ahead of its own (the MFMA takes 16 cycles, an LDS read about
      // 100: left to itself the compiler read 3 ahead and each MFMA waited)
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const bf16x4 v = vf[i % kWVAhead];
        if (i + kWVAhead < 32) vf[i % kWVAhead] = lds_read_tr16(vb + 32 * (i + kWVAhead));
        oacc[i] = mfma_16x16x16(pb, v, oacc[i]);
        __builtin_amdgcn_sched_barrier(0);  // keep the interleave
      }
    }
    if (ns > 0 && jn < nq) qloaded = jn;
    wave_epilogue(p, qb_of(j), qm_of(j), m_run, l_run, oacc);
    m_run = -INFINITY;
    l_run = 0.f;
#pragma unroll
    for (int blk = 0; blk < 32; ++blk) oacc[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

// ============================================================================
// shared-row tile kernel
// ============================================================================
// LDS row layout: a gathered row is 1 KiB stored at a 1072-byte pitch, and
// every K/V read of a lane is its base address plus a compile-time offset.
// Measured on gfx950 (4 waves per CU, 8 reads in flight per wave), for this
// kernel's read patterns: ds_read_b128 of K reaches 248 B/clk per CU at 1040,
// 1072 or 1104 and 128 at 1056; the transposing ds_read_b64_tr_b16 of V
// reaches 253 B/clk at 1056, 1072 or 1104 and 128 at 1040.
constexpr int kTilePitch = kRowBytes + 48;

// Work split of a tile step (64 union rows x 8 queries x 16 heads):
//  * S^T = K . Q^T and the softmax: wave w owns two queries (32 score
//    columns): their Q^T (128 VGPRs), softmax state and sums.
//      S^T block rb (rows 32rb..32rb+31) x the wave's 32 columns: lane
//      (l32, hi) holds column l32 (query 2w + l32/16, head l32 % 16) and rows
//      32rb + 8a + 4hi + b in register 4a + b.
//  * P goes to LDS as bf16 P[column][row] (one 144-byte line per column).
//  * O = P . V: wave w owns d = 128w..128w+127 of all 128 columns (16 blocks
//    of 32 x 32 fp32 in AGPRs). Each wave reads P (16 KiB) and its quarter of
//    V (16 KiB) per step instead of all of V (64 KiB).
//      accumulator 4k + db: rows are columns 32cb + 8(i/4) + 4hi + i%4 with
//      cb = (w + k) & 3 (register i; block k = 0 is the wave's own columns),
//      MFMA column l32 is d = 128w + 32db + l32.
// Barriers per step: one after each half of P is written (LDS only) and the
// gather's.
constexpr int kPPitch = 2 * kTileRows + 16;  // bytes per P column line
constexpr int kTileCols = kTQ * kHeads;      // 128 score columns
// K fragments of S^T = K . Q^T in flight: each ds_read_b128 is issued
// kKRing - 1 MFMAs before the MFMA that consumes it.
constexpr int kKRing = 6;
// The 16 row gathers of a wave's share of the next step are issued one per
// kDmaEvery MFMAs of S^T = K . Q^T. Every second MFMA of the first 32 (rows
// 0..31, before the softmax work joins the slots) measured 1 % faster than
// one per four spread over all 64.
constexpr int kDmaEvery = 2;
static_assert(kDmaEvery * 16 <= 2 * (kDim / 16), "the gathers fit in the S^T MFMAs");

struct TileSmem {
  uint8_t tile[2][kTileRows * kTilePitch];
  uint8_t p[kTileCols * kPPitch];
  _Float16 lc[2][kTQ * kTileRows];
  int abort;
};
// The tile kernel's work-groups either run a shared tile or, as per-query
// workers, query units: the two layouts share the LDS.
union TileQuerySmem {
  TileSmem t;
  QuerySmem q;
};

// The order entry of a shared tile t with nU union rows: its step count plus
// one above the tile (an all-masked tile has no step).
__device__ __forceinline__ int32_t shared_entry(int64_t t, int nU) {
  return int32_t(((1 + (nU + kTileRows - 1) / kTileRows) << kOrderTileBits) | int32_t(t));
}

// One shared tile, whose order entry is `entry` (a nonzero step key). It
// returns with every transfer it issued complete.
// kSkip: the pair-skipping form of the step (below, "Pair skipping"), for
// tiles whose query pairs often name no row of a 32-row half-step; the dense
// form otherwise. Their results are the same bits.
template <bool kSkip>
__device__ __forceinline__ void tile_run(const TileParams p, const int32_t entry, const int tid) {
  __shared__ __attribute__((aligned(16))) TileQuerySmem sm;
  auto& s_tile = sm.t.tile;
  auto& s_p = sm.t.p;
  auto& s_lc = sm.t.lc;
  auto& s_abort = sm.t.abort;

  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  const int64_t tile = entry & ((1 << kOrderTileBits) - 1);
  const int nsteps = (entry >> kOrderTileBits) - 1;
  const int64_t bi = tile / p.tiles_per_b;
  const int64_t q0 = (tile % p.tiles_per_b) * kTQ;
  const int qt = int(min(int64_t(kTQ), p.m - q0));
  if (nsteps == 0) {
    // no valid slot in any query of the tile: the sink takes all the mass
    __bf16* ob = p.o + bi * p.so_b + q0 * p.so_m;
    for (int i = tid; i < qt * kHeads * (kDim / 8); i += kThreads) {
      const int qh = i / (kDim / 8);
      bf16x8 z;
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] = static_cast<__bf16>(0.f);
      *reinterpret_cast<bf16x8*>(ob + int64_t(qh >> 4) * p.so_m + int64_t(qh & 15) * p.so_h +
                                 8 * (i % (kDim / 8))) = z;
    }
    if (p.lse != nullptr && tid < qt * kHeads)  // ln(exp(sink)) = sink, -inf without one
      p.lse[bi * p.sl_b + (q0 + (tid >> 4)) * p.sl_m + int64_t(tid & 15) * p.sl_h] =
          p.sink[tid & 15];
    return;
  }

  const int qw = 2 * wave + (l32 >> 4);  // this lane's query within the tile
  const int hh = l32 & 15;                // and head
  const uint32_t* urows = p.row_off + tile * p.cap;
  // The first step's union offsets are loaded before Q: loads complete in
  // order, so the first gather then waits for them alone, not for the
  // 32 KiB of Q per wave, which arrives while the rows are gathered.
  const int rows0 = int(urows[wave * kRowsPerWave + (lane & 15)]);
  asm volatile("" ::: "memory");  // keep Q's loads after it
  // Every lane loads (a lane past the tile's last query reads query 0 and
  // zeroes it), so the loads are not under a branch and the first gather's
  // wait counts only them as younger.
  bf16x8 qf[kDim / 16];
  {
    const __bf16* qrow = p.q + bi * p.sq_b + (q0 + (qw < qt ? qw : 0)) * p.sq_m +
                         int64_t(hh) * p.sq_h + 8 * hi;
#pragma unroll
    for (int s = 0; s < kDim / 16; ++s) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 16 * s);
  }

  const _Float16* ulc = p.lcnt + tile * p.cap * kTQ;
  const uint8_t* kvb = reinterpret_cast<const uint8_t*>(p.kv + bi * p.skv_b);
  // LDS address of this wave's first tile row in buffer 0
  const uint32_t lds_rows = __builtin_amdgcn_readfirstlane(uint32_t(
      reinterpret_cast<uintptr_t>((lds_u8_t*)&s_tile[0][wave * kRowsPerWave * kTilePitch])));

  // Union rows of a step: lane i (< 16) of wave w holds the byte offset of
  // row 16w + i. The gather reads them back with readlane, so each row's
  // address is a scalar base.
  auto step_rows = [&](int step) -> int {
    return int(urows[step * kTileRows + wave * kRowsPerWave + (lane & 15)]);
  };
  // One 1 KiB row into LDS row 16w + i (lane l moves bytes 16l..16l+15).
  auto dma_row = [&](int rows_v, int i, int buf) {
    const uint32_t off = uint32_t(__builtin_amdgcn_readlane(rows_v, i));
    lds_dma_row(kvb + off, 16 * lane,
                lds_rows + uint32_t(buf * kTileRows * kTilePitch + i * kTilePitch));
  };
  // The 1 KiB of log2 multiplicities of a step (wave 0).
  auto dma_counts = [&](int step, int buf) {
    if (wave == 0) lds_dma16_async(ulc + step * (kTQ * kTileRows) + 8 * lane, &s_lc[buf][0]);
  };

  float m_run = -INFINITY;  // reference max of column l32 (log2 domain)
  float l_run = 0.f;        // this lane's share of the column's sum
  f32x16 oacc[kDim / 32];   // [4k + db], column block (wave + k) & 3
#pragma unroll
  for (int nb = 0; nb < kDim / 32; ++nb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) oacc[nb][i] = 0.f;
    asm volatile("" : "+a"(oacc[nb]));  // O lives in AGPRs (MFMA C/D only)
  }

#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) dma_row(rows0, i, 0);
  dma_counts(0, 0);
  if (qw >= qt) {
#pragma unroll
    for (int s = 0; s < kDim / 16; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] = static_cast<__bf16>(0.f);
  }
  int rows_next = step_rows(min(1, nsteps - 1));
  if (tid == 0) s_abort = 0;
  dma_barrier();

  // K operand: lane reads row 32rb + l32, bytes 32s + 16hi.
  const int koff = l32 * kTilePitch + 16 * hi;
  // V operand (B of O = P . V): 16-lane group G, lane j reads row
  // 16kb + 8(G>>1) + j/4 (and 4 rows on), d = 128w + 32db + 16(G&1) + 4(j&3)
  // .. +3, and receives d = 128w + 32db + 16(G&1) + j over 4 rows.
  const int G = lane >> 4;
  const int j = lane & 15;
  const int voff =
      (8 * (G >> 1) + (j >> 2)) * kTilePitch + 2 * (128 * wave + 16 * (G & 1) + 4 * (j & 3));
  // P operand (A): for accumulator block k the lane reads column
  // 32 * ((w + k) & 3) + l32, rows 16kb + 8hi .. +7. Block 0 is the wave's own
  // columns, which it can read before the other waves' P is in LDS.
  const uint8_t* prd[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    prd[k] = s_p + (32 * ((wave + k) & 3) + l32) * kPPitch + 16 * hi;
  // P store: this lane's column 32w + l32, rows 32rb + 8a + 4hi .. +3.
  uint8_t* pwrite = s_p + (32 * wave + l32) * kPPitch + 8 * hi;

  // Softmax of one 32-row half of a step, cut into slots that ride between
  // MFMAs. Each slot's instructions are independent of one another, so none
  // of them waits on the previous one's result and holds up the next MFMA:
  //  * slots 0..7 turn two scores each into x = s * scale + log2 c (-inf for
  //    rows the query does not name); slots 1..8 fold the previous slot's two
  //    into the column max;
  //  * slot 9 merges the max of the lane pair, slot 10 checks / sets the
  //    column's reference;
  //  * element e is shifted (x - m) in slot 11 + e, exponentiated in slot
  //    12 + e and added to the column sum / packed to bf16 in slot 13 + e;
  //    P is stored every fourth element.
  // (v_dot2 forms of the sum stall the MFMAs they are interleaved with on
  // gfx950: plain adds.)
  constexpr int kSmSlots = 29;
  bool abort_any = false;  // wave-uniform: a column jumped above its reference
  auto sm_slot = [&](int k, f32x16& x, const f16x4(&lc)[4], int rb, float& mx, float& mref,
                     float& psum, bf16x4& pk) {
    if (k >= 1 && k <= 8)
      mx = fmaxf(mx, fmaxf(x[2 * k - 2], x[2 * k - 1]));  // v_max3
    if (k < 8) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int e = 2 * k + t;
        x[e] = fmaf(x[e], p.scale_log2, static_cast<float>(lc[e >> 2][e & 3]));
      }
    } else if (k == 9) {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                       false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));  // -inf: no row in the half
    } else if (k == 10) {
      // Fixed reference: a column keeps the max of its first non-empty half.
      // A later score more than kTileMaxJump above it would need O rescaled;
      // the tile then runs its queries per query instead.
      abort_any |= __any(m_run != -INFINITY && mx > m_run + kTileMaxJump) != 0;
      if (m_run == -INFINITY) m_run = mx;
      mref = m_run == -INFINITY ? 0.f : m_run;  // column still empty
    } else if (k < kSmSlots) {
      const int c = k - 13;  // sum and pack
      if (c >= 0 && c < 16) {
        psum += x[c];
        asm volatile("" : "+v"(psum));  // keep the sum in its slot (not sunk to the loop end)
        pk[c & 3] = static_cast<__bf16>(x[c]);
        if ((c & 3) == 3) *reinterpret_cast<bf16x4*>(pwrite + 2 * (32 * rb + 8 * (c >> 2))) = pk;
      }
      const int b = k - 12;  // c * 2^(s - m); 0 if masked
      if (b >= 0 && b < 16) x[b] = __builtin_amdgcn_exp2f(x[b]);
      const int a = k - 11;
      if (a >= 0 && a < 16) x[a] -= mref;
    }
  };
  static_assert(kSmSlots <= 32, "the softmax of a half fits in 32 MFMA slots");

  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const uint8_t* tb = s_tile[buf];
    const _Float16* lb = s_lc[buf];
    const int nxt = min(step + 1, nsteps - 1);  // the last step refetches itself: harmless

    // log2 multiplicities of this lane's rows in its query: rows
    // 32rb + 8a + 4hi + (0..3)
    f16x4 lc0[4], lc1[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      lc0[a] = *reinterpret_cast<const f16x4*>(&lb[qw * kTileRows + 8 * a + 4 * hi]);
      lc1[a] = *reinterpret_cast<const f16x4*>(&lb[qw * kTileRows + 32 + 8 * a + 4 * hi]);
    }
    // Pair skipping: the multiplicities of all 8 queries, 8 rows per lane
    // (lane l: query l / 8, rows 8 (l % 8) ..), to tell which query pairs
    // name a row of each half of the step.
    uint4 lca;
    if constexpr (kSkip)
      lca = *reinterpret_cast<const uint4*>(&lb[(lane >> 3) * kTileRows + 8 * (lane & 7)]);
    uint32_t act0 = 0xFu, act1 = 0xFu;  // bit j: queries 2j, 2j + 1 name a row of rows 0..31 / 32..63
    // A named row's multiplicity is log2(count) >= 0 (sign bit clear), an
    // unnamed one -inf (sign bit set).
    auto pair_activity = [&]() {
      const uint32_t all = lca.x & lca.y & lca.z & lca.w;
      const uint64_t named = __ballot((all & 0x80008000u) != 0x80008000u);
      act0 = act1 = 0u;
#pragma unroll
      for (int j = 0; j < kTQ / 2; ++j) {
        act0 |= (named & (0x0F0Full << (16 * j))) != 0ull ? 1u << j : 0u;
        act1 |= (named & (0xF0F0ull << (16 * j))) != 0ull ? 1u << j : 0u;
      }
    };

    // ---- S^T = K . Q^T, rows 0..31 then 32..63; the softmax of rows 0..31 runs
    // between the MFMAs of rows 32..63. All 16 rows of this wave's share of the
    // next step are gathered between the MFMAs of rows 0..31, so they have the
    // rest of the step to land.
    f32x16 sacc0, sacc1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sacc0[i] = 0.f;
      sacc1[i] = 0.f;
    }
    // Pair skipping also skips S^T: wave w computes S^T for pair w only, so
    // a half of the step that the pair does not name takes none of its 32
    // MFMAs (its scores would all be -inf: p = 0, the sums and the reference
    // unchanged, and P.V skips the block). Both halves named: the dense
    // chain.
    bool sthalf0 = true, sthalf1 = true;
    if constexpr (kSkip) {
      pair_activity();
      sthalf0 = ((act0 >> wave) & 1u) != 0u;
      sthalf1 = ((act1 >> wave) & 1u) != 0u;
    }
    {
      const uint8_t* kr = tb + koff;
      bf16x8 kf[kKRing];
      auto kread = [&](int i, int slot) {
        kf[slot] =
            *reinterpret_cast<const bf16x8*>(kr + (i >> 5) * 32 * kTilePitch + 32 * (i & 31));
      };
      float mx = -INFINITY, mref = 0.f, psum = 0.f;
      bf16x4 pk;
      // S^T over the MFMAs [kLo, kHi) of the 64 (32 per half). The gathers ride
      // the first half's MFMAs (when the chain starts at 0); the softmax of rows
      // 0..31 rides the second half's when the chain is whole.
      auto st_chain = [&](auto lo_c, auto hi_c) {
        constexpr int kLo = decltype(lo_c)::value, kHi = decltype(hi_c)::value;
#pragma unroll
        for (int i = kLo; i < kLo + kKRing - 1; ++i) kread(i, i % kKRing);
#pragma unroll
        for (int i = kLo; i < kHi; ++i) {
          if (i + kKRing - 1 < kHi) kread(i + kKRing - 1, (i + kKRing - 1) % kKRing);
          if (i < kDim / 16)
            sacc0 = mfma_32x32x16(kf[i % kKRing], qf[i], sacc0);
          else
            sacc1 = mfma_32x32x16(kf[i % kKRing], qf[i - kDim / 16], sacc1);
          if (kLo == 0 && i % kDmaEvery == kDmaEvery - 1 && i / kDmaEvery < kRowsPerWave)
            dma_row(rows_next, i / kDmaEvery, buf ^ 1);
          if (kLo == 0 && i == 1) dma_counts(nxt, buf ^ 1);
          if (kLo == 0 && kHi == 2 * (kDim / 16) && i >= kDim / 16)
            sm_slot(i - kDim / 16, sacc0, lc0, 0, mx, mref, psum, pk);

          __builtin_amdgcn_sched_barrier(0);  // keep the interleave
        }
      };
      using I0 = std::integral_constant<int, 0>;
      using I32 = std::integral_constant<int, kDim / 16>;
      using I64 = std::integral_constant<int, 2 * (kDim / 16)>;
      if (!kSkip || (sthalf0 && sthalf1)) {
        st_chain(I0{}, I64{});
      } else {
        if (sthalf0) {
          st_chain(I0{}, I32{});
#pragma unroll
          for (int j = 0; j < kSmSlots; ++j) sm_slot(j, sacc0, lc0, 0, mx, mref, psum, pk);
        } else {
#pragma unroll
          for (int i = 0; i < kRowsPerWave; ++i) dma_row(rows_next, i, buf ^ 1);
          dma_counts(nxt, buf ^ 1);
        }
        if (sthalf1) st_chain(I32{}, I64{});
      }
      l_run += psum;
    }
    rows_next = step_rows(min(step + 2, nsteps - 1));

    // ---- O += P . V over 32 rows (k-blocks kb0, kb0 + 1): per k-block 4 P
    // fragments (b128, the second k-block's read during the first) and 4 V
    // fragments (2 transposing reads each) read two ahead into a 3-slot ring;
    // each V fragment feeds 4 MFMAs. `sync()` is the barrier that makes every
    // wave's P of these rows visible: the first V fragments and the wave's own
    // P columns are read before it. `extra(j)` is VALU work issued after the
    // j-th of the 32 MFMAs, while it executes.
    auto pv_half = [&](int kb0, auto&& sync, auto&& extra) {
      bf16x8 af[2][4];
      bf16x8 vf[3];
      auto pread_k = [&](int kb, int slot, int k) {
        af[slot][k] = *reinterpret_cast<const bf16x8*>(prd[k] + 32 * kb);
      };
      auto vread = [&](int n, int slot) {
        const uint8_t* v0 = tb + voff + 16 * (kb0 + (n >> 2)) * kTilePitch + 64 * (n & 3);
        const bf16x4 lo = lds_read_tr16(v0);
        const bf16x4 up = lds_read_tr16(v0 + 4 * kTilePitch);
        vf[slot] = __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7);
      };
      vread(0, 0);
      vread(1, 1);
      pread_k(kb0, 0, 0);
      sync();
#pragma unroll
      for (int k = 1; k < 4; ++k) pread_k(kb0, 0, k);
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int kb = n >> 2;
        const int db = n & 3;
        if (n + 2 < 8) vread(n + 2, (n + 2) % 3);
        if (n == 0) {
#pragma unroll
          for (int k = 0; k < 4; ++k) pread_k(kb0 + 1, 1, k);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          mfma_agpr(oacc[4 * k + db], af[kb][k], vf[n % 3]);
          extra(4 * n + k);
          __builtin_amdgcn_sched_barrier(0);  // one MFMA per slot, reads ahead in order
        }
      }
    };

    int abort_seen = 0;
    if constexpr (!kSkip) {
      // ---- O += P . V, rows 0..31, with the softmax of rows 32..63 ---------------
      {
        float mx = -INFINITY, mref = 0.f, psum = 0.f;
        bf16x4 pk;
        pv_half(0, [&]() { lds_barrier(); },  // P rows 0..31 of every column are in LDS
                [&](int j) { sm_slot(j, sacc1, lc1, 1, mx, mref, psum, pk); });
        l_run += psum;
      }

      // ---- O += P . V, rows 32..63 -----------------------------------------------
      pv_half(2,
              [&]() {
                if (abort_any) s_abort = 1;
                lds_barrier();  // P rows 32..63 are in LDS; every abort of this step is set
                abort_seen = s_abort;
              },
              [](int) {});
    } else {
      // ---- Pair skipping: the softmax of rows 32..63 runs on its own (not
      // interleaved with MFMAs), so that P of all 64 rows is in LDS after one
      // barrier. Then O += P . V over the step's 64 rows, one 32-row half and
      // one column block (query pair, 2 k-blocks x 4 d-blocks = 8 MFMAs) at a
      // time: a block whose pair names no row of the half skips its MFMAs at
      // the cost of one branch (its P is all zero there; with the dense form's
      // interleaving such branches would sit around the softmax, and the
      // compiler then spills its state). Per accumulator the MFMAs run in the
      // dense form's order, so the sums are the same.
      if (sthalf1) {  // (a half the pair does not name has no P to read)
        float mx = -INFINITY, mref = 0.f, psum = 0.f;
        bf16x4 pk;
#pragma unroll
        for (int j = 0; j < kSmSlots; ++j) sm_slot(j, sacc1, lc1, 1, mx, mref, psum, pk);
        l_run += psum;
      }
      auto pread = [&](bf16x8 (&af)[2][4], int kb0) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int k = 0; k < 4; ++k)
            af[kb][k] = *reinterpret_cast<const bf16x8*>(prd[k] + 32 * (kb0 + kb));
      };
      auto vread = [&](bf16x8 (&vf)[8], int kb0) {
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const uint8_t* v0 = tb + voff + 16 * (kb0 + (n >> 2)) * kTilePitch + 64 * (n & 3);
          const bf16x4 lo = lds_read_tr16(v0);
          const bf16x4 up = lds_read_tr16(v0 + 4 * kTilePitch);
          vf[n] = __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7);
        }
      };
      auto pv_blocks = [&](const bf16x8 (&af)[2][4], const bf16x8 (&vf)[8], uint32_t act) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (((act >> ((wave + k) & 3)) & 1u) != 0) {
#pragma unroll
            for (int n = 0; n < 8; ++n) {
              mfma_agpr(oacc[4 * k + (n & 3)], af[n >> 2][k], vf[n]);
              __builtin_amdgcn_sched_barrier(0);  // one MFMA per slot, in order
            }
          }
        }
      };
      bf16x8 vf[8], af[2][4];
      vread(vf, 0);  // V is in LDS since the gather barrier
      if (abort_any) s_abort = 1;
      lds_barrier();  // P rows 0..63 are in LDS; every abort of this step is set
      abort_seen = s_abort;
      pread(af, 0);
      pv_blocks(af, vf, __builtin_amdgcn_readfirstlane(act0));
      vread(vf, 2);
      pread(af, 2);
      pv_blocks(af, vf, __builtin_amdgcn_readfirstlane(act1));
    }

    dma_barrier();  // every wave's prefetch has landed; P and this tile are free
    if (abort_seen != 0) {  // uniform: every wave read it after the same barrier
      // The tile's queries run per query here (online rescale); nothing of
      // the tile was written and no transfer is in flight.
      for (int j = 0; j < qt; ++j) {
        query_unit<4>(p.fwd, bi * p.m + q0 + j, sm.q);
        __syncthreads();
      }
      return;
    }
  }

  // ---- epilogue: column sums, sink fold, bf16 store -----------------------------
  mfma_agpr_drain();
  // The owner lane of a column computes its normalizer; P's LDS lines are free
  // after the last barrier and carry the 128 normalizers to every wave.
  float* s_f = reinterpret_cast<float*>(s_p);
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run),
                                                     __float_as_uint(l_run), false, false);
    const float lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    float lse;
    const float f = sink_fold(m_run, lt, p.sink[hh] * kLog2e, lse);
    if (hi == 0) {
      s_f[32 * wave + l32] = f;
      if (p.lse != nullptr && qw < qt)
        p.lse[bi * p.sl_b + (q0 + qw) * p.sl_m + int64_t(hh) * p.sl_h] = lse;
    }
  }
  lds_barrier();
  // Nontemporal: the tile's o is not read again by this launch, and its
  // 128 KiB would otherwise take L2 lines from the other tiles' rows.
  // Column c = 32kk + 8a + 4hi + b is o row (query c / 16, head c % 16): a
  // per-lane base (hi, d) plus a wave-uniform offset, so the row addresses
  // are scalar arithmetic. Columns b and b + 1 share one conversion; the
  // upper half is stored by the d16_hi form.
  __bf16* const lbase = p.o + bi * p.so_b + q0 * p.so_m + int64_t(4 * hi) * p.so_h + 128 * wave + l32;
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int kk = (wave + k) & 3;
      const int col0 = 32 * kk + 8 * a + 4 * hi;  // columns col0 .. col0 + 3
      const f32x4 fs = *reinterpret_cast<const f32x4*>(&s_f[col0]);
      const int q2 = 2 * kk + (a >> 1);           // wave-uniform
      if (q2 < qt) {
        const int64_t uoff = int64_t(q2) * p.so_m + int64_t(8 * (a & 1)) * p.so_h;
#pragma unroll
        for (int b = 0; b < 4; b += 2) {
          __bf16* r0 = lbase + uoff + int64_t(b) * p.so_h;
          __bf16* r1 = r0 + p.so_h;
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const f32x2_t f2 = {oacc[4 * k + db][4 * a + b] * fs[b],
                                oacc[4 * k + db][4 * a + b + 1] * fs[b + 1]};
            const bf16x2_t h2 = __builtin_convertvector(f2, bf16x2_t);
            __builtin_nontemporal_store(h2[0], &r0[32 * db]);
            __builtin_nontemporal_store(h2[1], &r1[32 * db]);
          }
        }
      }
    }
}

// kScan = false: work-group i runs entry order[i] (one work-group per tile;
// those of per-query tiles return at once), or the placed launch's tile i.
// kScan = true (short-query plans, whose per-query tiles run in
// sa_fwd_wave_kernel, so that most tiles are usually per-query): a grid of G
// work-groups, one per CU, where work-group b walks the tiles b, b + G,
// b + 2G, ... and runs the shared ones; no order is made. One work-group per
// tile at one per CU (by LDS) made a launch whose 8 192 tiles were all
// per-query take 14.8 us, its work-groups each only reading the order entry.
template <bool kSkip, bool kScan>
__global__ void __launch_bounds__(kThreads, 1) sa_fwd_tile_kernel(const TileParams p) {
  if constexpr (kScan) {
    const int64_t G = gridDim.x;
    const int lane = threadIdx.x & 63;
    for (int64_t t0 = blockIdx.x; t0 < p.ntiles; t0 += 64 * G) {
      // lane i tests tile t0 + iG; every wave reads the same modes, so the
      // mask, and with it the loop below, is the same in all four
      const int64_t tl = t0 + lane * G;
      const bool sh = tl < p.ntiles && p.meta[tl * kMetaInts + 1] == kModeShared;
      uint64_t mask = __ballot(sh);
      while (mask != 0) {
        const int64_t t = t0 + int64_t(__builtin_ctzll(mask)) * G;
        mask &= mask - 1;
        const int nU = __builtin_amdgcn_readfirstlane(p.meta[t * kMetaInts]);
        const __attribute__((address_space(4))) TileParams* pk =
            (const __attribute__((address_space(4))) TileParams*)__builtin_amdgcn_kernarg_segment_ptr();
        int tid = threadIdx.x;
        asm volatile("" : "+s"(pk), "+v"(tid));
        tile_run<kSkip>(*(const TileParams*)(const void*)pk, shared_entry(t, nU), tid);
        __syncthreads();  // the next tile's gathers overwrite this one's LDS
      }
    }
  } else {
    int32_t entry;
    if (p.placed) {
      // At most one tile per CU and at least one per two, all starting at
      // once: the order kernel's XCD-local placement, computed here
      // (work-group i runs on XCD i % 8; XCD x takes the x-th eighth of the
      // tiles in tile order).
      const int n = int(p.ntiles);
      const int x = int(blockIdx.x) % kXcds;
      int first = 0;
      for (int y = 0; y < x; ++y) first += (n - y + kXcds - 1) / kXcds;
      const int t = first + int(blockIdx.x) / kXcds;
      const int32_t* mt = p.meta + int64_t(t) * kMetaInts;
      const int nU = __builtin_amdgcn_readfirstlane(mt[0]);
      const bool shared = __builtin_amdgcn_readfirstlane(mt[1]) == kModeShared;
      entry = shared ? shared_entry(t, nU) : 0;
    } else {
      entry = p.order[blockIdx.x];  // one load: tile and step count
    }
    // a per-query tile: its queries run in the per-query launch
    if ((entry >> kOrderTileBits) == 0) return;
    tile_run<kSkip>(p, entry, threadIdx.x);
  }
}

// ============================================================================
// split-topk combine: one 64-thread work-group per (query, head)
// ============================================================================
// Parts are read in batches of kCombineBatch, every load of a batch issued
// before any is used, and merged with a running max (the accumulators are
// rescaled when a batch raises it), so a query costs one memory latency per
// batch.
constexpr int kCombineBatch = 8;

__global__ void __launch_bounds__(64) sa_combine_kernel(const CombineParams p) {
  const int64_t qid = blockIdx.x / kHeads;
  const int h = int(blockIdx.x % kHeads);
  const int64_t bi = qid / p.m;
  const int64_t mi = qid % p.m;
  const int d0 = threadIdx.x * 8;
  const float* part = p.part + qid * p.nsplit * kPartFloats;

  float M = -INFINITY;
  float L = 0.f;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (int s0 = 0; s0 < p.nsplit; s0 += kCombineBatch) {
    float ms[kCombineBatch], ls[kCombineBatch];
    float4 v0[kCombineBatch], v1[kCombineBatch];
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const int sp = min(s0 + u, p.nsplit - 1);  // past the end: re-read the last part, weight 0
      const float* ps = part + sp * kPartFloats;
      ms[u] = ps[h];
      ls[u] = ps[kHeads + h];
      const float4* po = reinterpret_cast<const float4*>(ps + 2 * kHeads + h * kDim + d0);
      v0[u] = po[0];
      v1[u] = po[1];
    }
    float Mb = M;
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      if (s0 + u >= p.nsplit) ms[u] = -INFINITY;
      Mb = fmaxf(Mb, ms[u]);
    }
    if (Mb != M) {  // the batch raised the max: rescale (M = -inf: nothing merged yet)
      const float r = M == -INFINITY ? 0.f : exp2f(M - Mb);
      L *= r;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= r;
      M = Mb;
    }
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      // a part without a valid slot (or past the end) has weight 0; its
      // partials are never inf or NaN, so 0 * them is 0
      const float w = ms[u] == -INFINITY ? 0.f : exp2f(ms[u] - M);
      L += w * ls[u];
      acc[0] += w * v0[u].x;
      acc[1] += w * v0[u].y;
      acc[2] += w * v0[u].z;
      acc[3] += w * v0[u].w;
      acc[4] += w * v1[u].x;
      acc[5] += w * v1[u].y;
      acc[6] += w * v1[u].z;
      acc[7] += w * v1[u].w;
    }
  }
  float lse;
  const float f = sink_fold(M, L, p.sink[h] * kLog2e, lse);
  if (p.lse != nullptr && threadIdx.x == 0)
    p.lse[bi * p.sl_b + mi * p.sl_m + int64_t(h) * p.sl_h] = lse;
  bf16x8 v;
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = static_cast<__bf16>(acc[k] * f);
  *reinterpret_cast<bf16x8*>(p.o + bi * p.so_b + mi * p.so_m + int64_t(h) * p.so_h + d0) = v;
}

// ============================================================================
// merge of partial (o, lse) results: one wave64 per (b, m, h)
// ============================================================================
// lse = ln(sum_i exp(lse_i) + exp(sink)), o = sum_i exp(lse_i - lse) o_i, the
// natural-log form of the split-topk combine (track-01/notes.md:32-41). Each
// lane owns 8 consecutive d of every 512-wide chunk.
__global__ void __launch_bounds__(256) sa_merge_kernel(const MergeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= p.b * p.m * p.h) return;
  const int64_t hi = row % p.h;
  const int64_t mi = (row / p.h) % p.m;
  const int64_t bi = row / (p.h * p.m);
  const float* lp = p.lse_parts + bi * p.slp_b + mi * p.slp_m + hi * p.slp_h;
  const float sink = p.sink != nullptr ? p.sink[hi] : -INFINITY;
  float mx = sink;
  for (int64_t i = 0; i < p.n; ++i) mx = fmaxf(mx, lp[i * p.slp_n]);
  float lse = -INFINITY;
  if (mx != -INFINITY) {
    float sum = expf(sink - mx);
    for (int64_t i = 0; i < p.n; ++i) sum += expf(lp[i * p.slp_n] - mx);
    lse = mx + logf(sum);
  }
  if (p.lse != nullptr && lane == 0) p.lse[bi * p.sl_b + mi * p.sl_m + hi * p.sl_h] = lse;
  const __bf16* op = p.o_parts + bi * p.sop_b + mi * p.sop_m + hi * p.sop_h;
  __bf16* orow = p.o + bi * p.so_b + mi * p.so_m + hi * p.so_h;
  for (int64_t d0 = 8 * lane; d0 < p.d; d0 += 512) {
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = 0.f;
    if (lse != -INFINITY) {
      for (int64_t i = 0; i < p.n; ++i) {
        const float li = lp[i * p.slp_n];
        if (li == -INFINITY) continue;  // a part without mass: its o is ignored
        const float w = expf(li - lse);
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(op + i * p.sop_n + d0);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += w * static_cast<float>(v[k]);
      }
    }
    bf16x8 out;
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = static_cast<__bf16>(acc[k]);
    *reinterpret_cast<bf16x8*>(orow + d0) = out;
  }
}

// ============================================================================
// head padding (calls with 1, 2, 4 or 8 heads)
// ============================================================================
// The kernels compute 16 heads. A call with fewer runs on a 16-head copy in
// its workspace: q padded with zero heads (and 16 sink entries), then the
// first h heads of the 16-head o (and lse) copied out. One thread per 8
// elements of a head's row; the padded heads' outputs are never read.
struct PadParams {
  const __bf16* q;     // [b, m, h, d], strides sq_*
  const float* sink;   // [h]
  __bf16* qp;          // [b * m, 16, d] contiguous
  float* sinkp;        // [16]
  const __bf16* op;    // [b * m, 16, d] contiguous
  const float* lsep;   // [b * m, 16] or null
  __bf16* o;           // [b, m, h, d], strides so_*
  float* lse;          // [b, m, h], strides sl_*, or null
  int64_t m, h, rows;  // rows = b * m * (16 for the pad, h for the unpad)
  int64_t sq_b, sq_m, sq_h, so_b, so_m, so_h, sl_b, sl_m, sl_h;
};

__global__ void __launch_bounds__(256) sa_pad_heads_kernel(const PadParams p) {
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t < kHeads) p.sinkp[t] = t < p.h ? p.sink[t] : 0.f;
  if (t >= p.rows * (kDim / 8)) return;
  const int64_t r = t / (kDim / 8);  // (b * m) * 16 + head
  const int c = int(t % (kDim / 8));
  const int64_t bm = r / kHeads, hh = r % kHeads;
  bf16x8 v;
  if (hh < p.h) {
    const int64_t bi = bm / p.m, mi = bm % p.m;
    v = *reinterpret_cast<const bf16x8*>(p.q + bi * p.sq_b + mi * p.sq_m + hh * p.sq_h + 8 * c);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<__bf16>(0.f);
  }
  *reinterpret_cast<bf16x8*>(p.qp + r * kDim + 8 * c) = v;
}

__global__ void __launch_bounds__(256) sa_unpad_heads_kernel(const PadParams p) {
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= p.rows * (kDim / 8)) return;
  const int64_t r = t / (kDim / 8);  // (b * m) * h + head
  const int c = int(t % (kDim / 8));
  const int64_t bm = r / p.h, hh = r % p.h;
  const int64_t bi = bm / p.m, mi = bm % p.m;
  const int64_t src = bm * kHeads + hh;
  *reinterpret_cast<bf16x8*>(p.o + bi * p.so_b + mi * p.so_m + hh * p.so_h + 8 * c) =
      *reinterpret_cast<const bf16x8*>(p.op + src * kDim + 8 * c);
  if (c == 0 && p.lse != nullptr) p.lse[bi * p.sl_b + mi * p.sl_m + hh * p.sl_h] = p.lsep[src];
}

// Compute units of the current device, cached per device ordinal.
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices];  // 0 = not yet queried (benign race: same value)

int current_cus(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SA_EHIP;
  if (dev >= 0 && dev < kMaxDevices) {
    const int cached = __atomic_load_n(&g_cus[dev], __ATOMIC_RELAXED);
    if (cached > 0) {
      *cus = cached;
      return SA_OK;
    }
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      v <= 0)
    return SA_EHIP;
  if (dev >= 0 && dev < kMaxDevices) __atomic_store_n(&g_cus[dev], v, __ATOMIC_RELAXED);
  *cus = v;
  return SA_OK;
}

// What forward() launches: every kernel of a call, or only the index plan.
enum class Launch { kCall, kPlanOnly };
int forward(const sa_args* a, hipStream_t stream, void* const* events, uint32_t* launched,
            Launch what = Launch::kCall);
// The same for 16 heads (forward() runs other head counts through it).
int forward16(const sa_args* a, hipStream_t stream, void* const* events, uint32_t* launched,
              Launch what);

}  // namespace

extern "C" {

int sa_abi_version(void) { return SA_ABI_VERSION; }

const char* sa_strerror(int code) {
  switch (code) {
    case SA_OK: return "ok";
    case SA_EINVAL: return "invalid argument (null pointer, size, stride, alignment or flags)";
    case SA_EUNSUPPORTED:
      return "unsupported shape (needs h = 1, 2, 4, 8 or a multiple of 16, and d = 512)";
    case SA_EWORKSPACE: return "workspace missing or too small";
    case SA_EHIP: return "HIP runtime error";
    case SA_ESCRATCH:
      return "the call needs more workspace than sa_forward_noalloc holds "
             "(SA_NOALLOC_SCRATCH_BYTES); use sa_forward with a workspace";
    default: return "unknown error";
  }
}

int sa_workspace_bytes(const sa_args* a, size_t* out_bytes) {
  if (out_bytes == nullptr) return SA_EINVAL;
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  *out_bytes = 0;
  if (a->b == 0 || a->m == 0) return SA_OK;
  int cus = 0;
  const int qrc = current_cus(&cus);
  if (qrc != SA_OK) return qrc;
  const size_t plan_bytes = sa::make_plan(a, cus).ws_bytes;
  *out_bytes = plan_bytes + sa::pad_layout(a, plan_bytes).bytes;
  return SA_OK;
}

int sa_forward(const sa_args* a, void* hip_stream) {
  return forward(a, static_cast<hipStream_t>(hip_stream), nullptr, nullptr);
}

int sa_forward_events(const sa_args* a, void* hip_stream, void* const* events,
                      uint32_t* launched) {
  if (launched != nullptr) *launched = 0u;
  return forward(a, static_cast<hipStream_t>(hip_stream), events, launched);
}

int sa_plan_indices(const sa_args* a, void* hip_stream) {
  return forward(a, static_cast<hipStream_t>(hip_stream), nullptr, nullptr, Launch::kPlanOnly);
}

int sa_merge(const sa_merge_args* a, void* hip_stream) {
  const int rc = sa::validate_merge(a);
  if (rc != SA_OK) return rc;
  const int64_t rows = a->b * a->m * a->h;
  if (rows == 0 || a->d == 0) return SA_OK;
  MergeParams p{};
  p.o_parts = static_cast<const __bf16*>(a->o_parts);
  p.lse_parts = a->lse_parts;
  p.sink = a->sink;
  p.o = static_cast<__bf16*>(a->o);
  p.lse = a->lse;
  p.n = a->n;
  p.b = a->b;
  p.m = a->m;
  p.h = a->h;
  p.d = a->d;
  p.sop_n = a->sop[0];
  p.sop_b = a->sop[1];
  p.sop_m = a->sop[2];
  p.sop_h = a->sop[3];
  p.slp_n = a->slp[0];
  p.slp_b = a->slp[1];
  p.slp_m = a->slp[2];
  p.slp_h = a->slp[3];
  p.so_b = a->so[0];
  p.so_m = a->so[1];
  p.so_h = a->so[2];
  p.sl_b = a->slse[0];
  p.sl_m = a->slse[1];
  p.sl_h = a->slse[2];
  hipLaunchKernelGGL(sa_merge_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(hip_stream), p);
  return hipGetLastError() == hipSuccess ? SA_OK : SA_EHIP;
}

}  // extern "C"

namespace {

// The launches of one call. With `events`, records events[2k] / events[2k+1]
// on the stream around kernel k (SA_KERNEL_*) and sets bit k of *launched.
// SA_FLAG_PLANNED skips the index kernels (their results are in the
// workspace); Launch::kPlanOnly runs only them.
// 16 heads: the kernels directly. 16 k heads: k calls on 16-head slices of
// q, sink, o and lse (strided views; the plan is head-independent, so an
// index plan serves every slice). 1, 2, 4 or 8 heads: a 16-head copy in the
// workspace after the plan's bytes (sa::pad_layout), zero-padded q in, the
// first h heads of o (and lse) out.
int forward(const sa_args* a, hipStream_t stream, void* const* events, uint32_t* launched,
            Launch what) {
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  if (a->h == kHeads || a->b == 0 || a->m == 0) return forward16(a, stream, events, launched, what);
  if (a->h > kHeads) {
    for (int64_t g = 0; g < a->h / kHeads; ++g) {
      sa_args s = *a;
      s.h = kHeads;
      s.q = static_cast<const __bf16*>(a->q) + g * kHeads * a->sq[2];
      s.o = static_cast<__bf16*>(a->o) + g * kHeads * a->so[2];
      s.sink = a->sink + g * kHeads;
      if (a->lse != nullptr) s.lse = a->lse + g * kHeads * a->slse[2];
      const int grc = forward16(&s, stream, events, launched, what);
      if (grc != SA_OK || what == Launch::kPlanOnly) return grc;
    }
    return SA_OK;
  }
  int cus = 0;
  const int qrc = current_cus(&cus);
  if (qrc != SA_OK) return qrc;
  const size_t plan_bytes = sa::make_plan(a, cus).ws_bytes;
  const sa::PadLayout pl = sa::pad_layout(a, plan_bytes);
  if (a->workspace == nullptr || a->workspace_bytes < plan_bytes + pl.bytes) return SA_EWORKSPACE;
  uint8_t* ws = static_cast<uint8_t*>(a->workspace);
  sa_args s = *a;
  s.h = kHeads;
  s.q = ws + pl.q_off;
  s.o = ws + pl.o_off;
  s.sink = reinterpret_cast<float*>(ws + pl.sink_off);
  s.lse = a->lse != nullptr ? reinterpret_cast<float*>(ws + pl.lse_off) : nullptr;
  const int64_t bm = a->b * a->m;
  s.sq[0] = a->m * kHeads * kDim;
  s.sq[1] = kHeads * kDim;
  s.sq[2] = kDim;
  s.sq[3] = 1;
  for (int i = 0; i < 4; ++i) s.so[i] = s.sq[i];
  s.slse[0] = a->m * kHeads;
  s.slse[1] = kHeads;
  s.slse[2] = 1;
  s.workspace_bytes = plan_bytes;
  if (what == Launch::kPlanOnly) return forward16(&s, stream, events, launched, what);
  PadParams pp{};
  pp.q = static_cast<const __bf16*>(a->q);
  pp.sink = a->sink;
  pp.qp = static_cast<__bf16*>(const_cast<void*>(s.q));
  pp.sinkp = const_cast<float*>(s.sink);
  pp.op = static_cast<const __bf16*>(s.o);
  pp.lsep = s.lse;
  pp.o = static_cast<__bf16*>(a->o);
  pp.lse = a->lse;
  pp.m = a->m;
  pp.h = a->h;
  pp.sq_b = a->sq[0];
  pp.sq_m = a->sq[1];
  pp.sq_h = a->sq[2];
  pp.so_b = a->so[0];
  pp.so_m = a->so[1];
  pp.so_h = a->so[2];
  pp.sl_b = a->slse[0];
  pp.sl_m = a->slse[1];
  pp.sl_h = a->slse[2];
  pp.rows = bm * kHeads;
  hipLaunchKernelGGL(sa_pad_heads_kernel, dim3(unsigned((pp.rows * (kDim / 8) + 255) / 256)),
                     dim3(256), 0, stream, pp);
  if (hipGetLastError() != hipSuccess) return SA_EHIP;
  const int frc = forward16(&s, stream, events, launched, what);
  if (frc != SA_OK) return frc;
  pp.rows = bm * a->h;
  hipLaunchKernelGGL(sa_unpad_heads_kernel, dim3(unsigned((pp.rows * (kDim / 8) + 255) / 256)),
                     dim3(256), 0, stream, pp);
  return hipGetLastError() == hipSuccess ? SA_OK : SA_EHIP;
}

int forward16(const sa_args* a, hipStream_t stream, void* const* events, uint32_t* launched,
              Launch what) {
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  if (a->b == 0 || a->m == 0) return SA_OK;
  int cus = 0;
  const int qrc = current_cus(&cus);
  if (qrc != SA_OK) return qrc;
  const sa::Plan plan = sa::make_plan(a, cus);
  if (plan.ws_bytes > 0 && (a->workspace == nullptr || a->workspace_bytes < plan.ws_bytes))
    return SA_EWORKSPACE;
  // Launches kernel k (SA_KERNEL_*) with its one parameter block. With the
  // caller's events, through hipExtLaunchKernel: events[2k] and events[2k+1]
  // then take the dispatch's own start and end timestamps (the ones a
  // kernel-trace profiler reads), not the stream position before and after
  // it, which would add the gap before the dispatch.
  auto run = [&](int k, const void* fn, dim3 grid, dim3 block, uint32_t lds, void* prm) -> int {
    void* kargs[] = {prm};
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (events != nullptr) {
      e0 = static_cast<hipEvent_t>(events[2 * k]);
      e1 = static_cast<hipEvent_t>(events[2 * k + 1]);
    }
    const hipError_t err =
        (e0 != nullptr || e1 != nullptr)
            ? hipExtLaunchKernel(fn, grid, block, kargs, lds, stream, e0, e1, 0)
            : hipLaunchKernel(fn, grid, block, kargs, lds, stream);
    if (err != hipSuccess || hipGetLastError() != hipSuccess) return SA_EHIP;
    if (launched != nullptr) *launched |= 1u << k;
    return SA_OK;
  };
  auto fn = [](auto kernel) { return reinterpret_cast<const void*>(kernel); };
  uint8_t* ws = static_cast<uint8_t*>(a->workspace);
  const float scale_log2 = a->scale * kLog2e;

  FwdParams p{};
  p.q = static_cast<const __bf16*>(a->q);
  p.kv = static_cast<const __bf16*>(a->kv);
  p.sink = a->sink;
  p.idx = a->idx;
  p.o = static_cast<__bf16*>(a->o);
  p.part = plan.nsplit > 1 ? reinterpret_cast<float*>(ws + plan.part_off) : nullptr;
  p.err = a->err_word;
  p.m = a->m;
  p.kv_len = a->kv_len;
  p.topk = a->topk;
  p.sq_b = a->sq[0];
  p.sq_m = a->sq[1];
  p.sq_h = a->sq[2];
  p.skv_b = a->skv[0];
  p.skv_n = a->skv[1];
  p.si_b = a->sidx[0];
  p.si_m = a->sidx[1];
  p.so_b = a->so[0];
  p.so_m = a->so[1];
  p.so_h = a->so[2];
  p.scale_log2 = scale_log2;
  p.lse = a->lse;
  p.sl_b = a->slse[0];
  p.sl_m = a->slse[1];
  p.sl_h = a->slse[2];
  p.nsplit = plan.nsplit;
  p.split_len = plan.split_len;
  p.nblocks = plan.units * plan.nsplit;
  // the wave kernel sorts its queries' rows when a batch's kv span exceeds an
  // XCD's L2 (from the shape alone, so every path of a call sorts alike)
  p.sort_wave = int64_t(a->kv_len) * a->skv[1] * 2 > kWaveSortBytes ? 1 : 0;

  // Short unsplit queries run one wave each (sa_fwd_wave_kernel): its list
  // holds 32-bit row offsets in a batch of kv. (Its epilogue's bf16 pair
  // stores need o 4-byte aligned: validate() asks for 16.)
  const bool wave_ok =
      what == Launch::kCall && plan.nsplit == 1 && a->topk <= kWaveMaxTopk && a->kv_len > 0 &&
      (a->kv_len - 1) * a->skv[1] * 2 + 2 * kDim <= int64_t(UINT32_MAX);

  // The per-query kernel; two work-groups per CU once there are at least two
  // per CU to run.
  auto launch_query = [&]() -> int {
    if (p.meta == nullptr && wave_ok)
      return run(SA_KERNEL_WAVE, fn(sa_fwd_wave_kernel),
                 dim3(unsigned((p.nblocks + kWQueries - 1) / kWQueries)), dim3(64), 0, &p);
    const dim3 grid(unsigned(p.nblocks)), block(kThreads);
    const bool two = p.nblocks >= 2 * int64_t(cus);
    const void* k = p.meta != nullptr
                        ? (two ? fn(sa_fwd_query_kernel<2, true>) : fn(sa_fwd_query_kernel<4, true>))
                        : (two ? fn(sa_fwd_query_kernel<2, false>) : fn(sa_fwd_query_kernel<4, false>));
    return run(SA_KERNEL_QUERY, k, grid, block, 0, &p);
  };

  if (plan.tiles) {
    IndexParams ip{};
    ip.idx = a->idx;
    ip.err = a->err_word;
    ip.meta = reinterpret_cast<int32_t*>(ws + plan.meta_off);
    ip.row_off = reinterpret_cast<uint32_t*>(ws + plan.rows_off);
    ip.lcnt = reinterpret_cast<_Float16*>(ws + plan.cnts_off);
    ip.m = a->m;
    ip.kv_len = a->kv_len;
    ip.topk = a->topk;
    ip.si_b = a->sidx[0];
    ip.si_m = a->sidx[1];
    ip.skv_n = a->skv[1];
    ip.tiles_per_b = plan.tiles_per_b;
    ip.cap = plan.tile_cap;
    ip.force = (a->flags & SA_FLAG_FORCE_TILES) ? 1 : 0;
    ip.vec4 = ((reinterpret_cast<uintptr_t>(a->idx) & 15u) == 0 && a->topk % 4 == 0 &&
               a->sidx[0] % 4 == 0 && a->sidx[1] % 4 == 0) ? 1 : 0;
    // from the shape alone, so that an index plan makes the plain call's modes
    ip.placed_regime = (2 * plan.ntiles >= cus && plan.ntiles <= cus) ? 1 : 0;
    int32_t* order = reinterpret_cast<int32_t*>(ws + plan.order_off);
    const bool planned = what == Launch::kCall && (a->flags & SA_FLAG_PLANNED) != 0;
    // Between half as many tiles as CUs and as many, every tile starts at
    // once and the order's placement is a formula: the tile kernel applies it
    // itself and no order is made. (Fewer tiles keep the order: with a CU or
    // more per tile, the longest-first order beats XCD placement. An index
    // plan always holds an order.)
    const bool placed = what == Launch::kCall && !planned && ip.placed_regime != 0;
    if (!planned) {
      const size_t lds = size_t(a->kv_len) * sizeof(unsigned long long);
      // long caches (one work-group per CU by LDS): twice the threads, half
      // the index vectors each
      const bool wide = a->kv_len >= kIdxWideKv;
      // small tiles: 256 threads, one round of 1 or 4 index vectors each
      const int64_t slots = kTQ * a->topk;
      const bool small1 = !wide && slots <= 256 * 4;
      const bool small4 = !wide && !small1 && slots <= kIdxSmallSlots;
      // long caches with short queries: the mode from a bitmap first
      const bool bits = wide && a->topk <= kWaveMaxTopk;
      const void* ik =
          bits     ? reinterpret_cast<const void*>(sa_tile_index_kernel<1024, 2, true>)
          : wide   ? reinterpret_cast<const void*>(sa_tile_index_kernel<1024, 2, false>)
          : small1 ? reinterpret_cast<const void*>(sa_tile_index_kernel<256, 1, false>)
          : small4 ? reinterpret_cast<const void*>(sa_tile_index_kernel<256, 4, false>)
                   : reinterpret_cast<const void*>(
                         sa_tile_index_kernel<kIdxThreadsNarrow, kIdxVecNarrow, false>);
      if (lds > 65536 &&
          hipFuncSetAttribute(ik, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) != hipSuccess)
        return SA_EHIP;
      const int irc = run(SA_KERNEL_INDEX, ik, dim3(unsigned(plan.ntiles)),
                          dim3(wide ? 1024 : (small1 || small4) ? 256 : kIdxThreadsNarrow),
                          uint32_t(lds), &ip);
      if (irc != SA_OK) return irc;
    }
    // The per-query launch: one work-group per tile runs the queries of a
    // per-query tile (the others return at once), and work-group 0 makes the
    // tile order when this call makes one (an index plan makes it in
    // sa_order_kernel instead, below; a short-query plan makes none, unless a
    // flag asks for the ordered tile launch).
    // (Running a placed call's per-query tiles in the tile kernel instead,
    // through the branch that reruns aborted tiles, makes the compiler spill
    // the kernel's 256 AGPR accumulators.)
    p.meta = ip.meta;
    p.tiles_per_b = plan.tiles_per_b;
    if (!planned && !placed) {
      p.ord.meta = ip.meta;
      p.ord.order = order;
      p.ord.ntiles = int(plan.ntiles);
      p.ord.cus = cus;
    }
    // An index plan makes only the union and the order, the latter in a
    // launch of its own. Short queries run per query as one wave each
    // (sa_fwd_wave_kernel), and their call makes no order: its tile launch
    // walks the tiles' modes itself (the scan form below), unless a flag
    // asks for the ordered launch.
    if (what == Launch::kPlanOnly)
      return run(SA_KERNEL_ORDER, fn(sa_order_kernel), dim3(1), dim3(kOrderThreads), 0, &p.ord);
    const bool scan = wave_ok && (a->flags & SA_FLAG_TILE_ORDERED) == 0;
    if (wave_ok) {
      if (!scan && p.ord.order != nullptr) {
        const int orc =
            run(SA_KERNEL_ORDER, fn(sa_order_kernel), dim3(1), dim3(kOrderThreads), 0, &p.ord);
        if (orc != SA_OK) return orc;
        p.ord.order = nullptr;
      }
      const int wrc = run(SA_KERNEL_WAVE, fn(sa_fwd_wave_kernel),
                          dim3(unsigned(plan.ntiles * (kTQ / kWQueries))), dim3(64), 0, &p);
      if (wrc != SA_OK) return wrc;
    } else {
      p.nblocks = plan.ntiles + (p.ord.order != nullptr ? 1 : 0);
      const int lrc = launch_query();
      if (lrc != SA_OK) return lrc;
    }

    TileParams tp{};
    tp.q = p.q;
    tp.kv = p.kv;
    tp.sink = a->sink;
    tp.o = p.o;
    tp.order = order;
    tp.row_off = ip.row_off;
    tp.lcnt = ip.lcnt;
    tp.m = a->m;
    tp.cap = plan.tile_cap;
    tp.tiles_per_b = plan.tiles_per_b;
    tp.sq_b = p.sq_b;
    tp.sq_m = p.sq_m;
    tp.sq_h = p.sq_h;
    tp.skv_b = p.skv_b;
    tp.skv_n = p.skv_n;
    tp.so_b = p.so_b;
    tp.so_m = p.so_m;
    tp.so_h = p.so_h;
    tp.scale_log2 = scale_log2;
    tp.lse = a->lse;
    tp.sl_b = a->slse[0];
    tp.sl_m = a->slse[1];
    tp.sl_h = a->slse[2];
    tp.ntiles = plan.ntiles;
    tp.fwd = p;
    tp.placed = placed ? 1 : 0;
    tp.meta = ip.meta;
    // One work-group per tile (those of per-query tiles return at once), or
    // after the wave launch one per CU that runs the shared tiles it finds.
    // The pair-skipping form when a row is named by fewer than one query of a
    // tile on average (high locality: 8 * 512 against 16 384 rows), unless a
    // flag forces one form.
    const bool skip = (a->flags & SA_FLAG_TILE_SKIP) != 0 ||
                      ((a->flags & SA_FLAG_TILE_DENSE) == 0 && kTQ * a->topk < a->kv_len);
    if (scan)
      return run(SA_KERNEL_TILE,
                 skip ? fn(sa_fwd_tile_kernel<true, true>) : fn(sa_fwd_tile_kernel<false, true>),
                 dim3(unsigned(std::min<int64_t>(plan.ntiles, cus))), dim3(kThreads), 0, &tp);
    return run(SA_KERNEL_TILE,
               skip ? fn(sa_fwd_tile_kernel<true, false>) : fn(sa_fwd_tile_kernel<false, false>),
               dim3(unsigned(plan.ntiles)), dim3(kThreads), 0, &tp);
  }
  if (what == Launch::kPlanOnly) return SA_OK;  // per-query plans keep no index state

  const int lrc = launch_query();
  if (lrc != SA_OK) return lrc;
  if (plan.nsplit > 1) {
    CombineParams c{};
    c.part = p.part;
    c.sink = a->sink;
    c.o = p.o;
    c.m = a->m;
    c.so_b = a->so[0];
    c.so_m = a->so[1];
    c.so_h = a->so[2];
    c.lse = a->lse;
    c.sl_b = a->slse[0];
    c.sl_m = a->slse[1];
    c.sl_h = a->slse[2];
    c.nsplit = plan.nsplit;
    const int crc = run(SA_KERNEL_COMBINE, fn(sa_combine_kernel),
                        dim3(unsigned(plan.units * kHeads)), dim3(64), 0, &c);
    if (crc != SA_OK) return crc;
  }
  return SA_OK;
}

}  // namespace

