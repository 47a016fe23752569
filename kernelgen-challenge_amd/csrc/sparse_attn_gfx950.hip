// sparse_attn_gfx950.hip -- MI355X (gfx950, CDNA4) kernels and C-ABI for
// top-k sparse attention with an attention sink, h = 16, d = 512, bf16 I/O.
//
// Math (track-01/reference/reference.py:24-40): for each query (b, m) and
// head h, s_t = scale * q[h] . kv[idx_t]; o[h] = sum_t softmax([s, sink[h]])_t
// * kv[idx_t] with the sink column dropped; o cast to bf16 (round to nearest
// even). -1 slots are excluded (track-01/submission.py:313-322).
//
// Kernel sa_fwd (one work-group of 4 wave64s per (query, topk part)):
//   1. compact the part's valid slot indices into LDS (order kept; bad
//      indices raise the error word and are dropped);
//   2. loop over tiles of 64 gathered rows, double-buffered in LDS: every row
//      is one coalesced 1 KiB wave load (64 lanes x 16 B) issued a full step
//      ahead into registers and written to the idle buffer at the end of the
//      step, so each row is read from memory once and shared by all 16 heads;
//   3. S^T = K . Q^T with v_mfma_f32_16x16x32_bf16: wave w owns tile rows
//      16w..16w+15 (M = rows, N = 16 heads, K = d = 512), Q^T held in
//      registers for the whole call;
//   4. online softmax in the log2 domain (scale * log2 e folded into the
//      scores, exp2): per-head tile max across the 4 waves through LDS, P
//      rounded to bf16 into LDS;
//   5. O += P . V with the same MFMA: wave w owns d columns 128w..128w+127
//      (M = 16 heads, N = d, K = 32 rows); V operands come from the same LDS
//      rows through ds_read_b64_tr_b16 transposing reads, so K and V share one
//      row-major copy;
//   6. epilogue: fold the sink (m_tot = max(m, sink), as the max over scores
//      and the sink in the reference's softmax) and store bf16, or store the
//      part's (max, sum, unnormalised O) for the combine kernel.
// Kernel sa_combine: merges the parts of one query with exp2(m_s - M)
// weights, folds the sink and stores bf16.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "sa_plan.h"
#include "sparse_attn.h"

namespace {

using sa::kDim;
using sa::kHeads;
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

static_assert(kListCap % kThreads == 0, "compaction split");
static_assert(kRowsPerWave == 16, "one 16-row MFMA block per wave");

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4_t;

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
  int nsplit;
  int64_t split_len;
  int64_t nblocks;      // grid size (units * nsplit)
};

struct CombineParams {
  const float* part;
  const float* sink;
  __bf16* o;
  int64_t m;
  int64_t so_b, so_m, so_h;
  int nsplit;
};

constexpr int64_t kPartFloats =
    (sa::kPartialMLBytes + sa::kPartialOBytes) / sizeof(float);

__device__ __forceinline__ f32x4 mfma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane j supplies the address
// of 4 consecutive bf16 (row j/4, columns 4*(j%4)..+3 of a 4 x 16 block) and
// receives column j of that block (4 values, one per row).
__device__ __forceinline__ bf16x4 lds_read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (lds_bf16x4_t*)((__attribute__((address_space(3))) uint8_t*)(p)));
}

__device__ __forceinline__ float wave_max16(float x) {  // over lanes n, n+16, n+32, n+48
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float wave_sum16(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// Logical unit for a work-group. Work-groups are dispatched round-robin over
// the 8 XCDs; this maps each XCD's work-groups to a contiguous run of units
// so neighbouring queries (which often share rows) share one L2.
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nblocks) {
  const int64_t per = nblocks / 8;
  if (bid >= per * 8) return bid;
  return (bid % 8) * per + bid / 8;
}

__global__ void __launch_bounds__(kThreads, 1) sa_fwd_kernel(const FwdParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t s_tile[2][kTileRows * kRowStride];
  __shared__ __attribute__((aligned(16))) int32_t s_list[kListCap];
  __shared__ __attribute__((aligned(16))) __bf16 s_p[kHeads * kTileRows];
  __shared__ float s_red[kWaves][kHeads];
  __shared__ int s_cnt[kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;   // MFMA column lane: head (S^T, P) or d (O)
  const int g = lane >> 4;   // MFMA k-group

  const int64_t unit = xcd_remap(blockIdx.x, p.nblocks);
  const int64_t qid = unit / p.nsplit;
  const int split = int(unit % p.nsplit);
  const int64_t bi = qid / p.m;
  const int64_t mi = qid % p.m;
  const int64_t s_begin = int64_t(split) * p.split_len;
  const int64_t s_end = min(p.topk, s_begin + p.split_len);

  // Q^T as the B operand of S^T = K . Q^T: lane (n, g) holds head n,
  // d = 32s + 8g .. 32s + 8g + 7 for k-step s.
  bf16x8 qf[kDim / 32];
  {
    const __bf16* qrow = p.q + bi * p.sq_b + mi * p.sq_m + int64_t(n) * p.sq_h + 8 * g;
#pragma unroll
    for (int s = 0; s < kDim / 32; ++s)
      qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s);
  }

  const __bf16* kvb = p.kv + bi * p.skv_b;
  const int32_t* irow = p.idx + bi * p.si_b + mi * p.si_m;

  float m_run = -INFINITY;  // running max (log2 domain) of head n
  float l_run = 0.f;        // this lane's share of the running sum of head n
  f32x4 oacc[kDBlocks];
#pragma unroll
  for (int i = 0; i < kDBlocks; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int64_t base = s_begin; base < s_end; base += kListCap) {
    const int cnt = int(min(int64_t(kListCap), s_end - base));
    __syncthreads();  // the previous batch is done with s_list
    // ---- 1. compaction of this batch's valid slots --------------------------
    int vals[kSlotsPerThread];
    int c = 0;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i) {
      const int sl = tid * kSlotsPerThread + i;
      int v = -1;
      if (sl < cnt) v = irow[base + sl];
      const bool ok = (v >= 0) && (int64_t(v) < p.kv_len);
      bad |= (!ok && v != -1);
      vals[i] = ok ? v : -1;
      c += ok ? 1 : 0;
    }
    if (bad && p.err != nullptr) atomicOr(p.err, 1);
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
    const int nsteps = (nvalid + kTileRows - 1) / kTileRows;

    // ---- 2. gather pipeline ---------------------------------------------------
    // wave w fetches tile rows 16w..16w+15; lane l moves bytes 16l..16l+15.
    bf16x8 pref[kRowsPerWave];
    auto fetch = [&](int step) {
#pragma unroll
      for (int i = 0; i < kRowsPerWave; ++i) {
        const int e = step * kTileRows + wave * kRowsPerWave + i;
        const int row = s_list[e < nvalid ? e : 0];  // tail rows: any valid row, masked
        pref[i] = *reinterpret_cast<const bf16x8*>(kvb + int64_t(row) * p.skv_n + 8 * lane);
      }
    };
    auto stash = [&](int buf) {
#pragma unroll
      for (int i = 0; i < kRowsPerWave; ++i)
        *reinterpret_cast<bf16x8*>(&s_tile[buf][(wave * kRowsPerWave + i) * kRowStride + 16 * lane]) =
            pref[i];
    };
    fetch(0);
    stash(0);
    __syncthreads();

    for (int step = 0; step < nsteps; ++step) {
      const uint8_t* tb = s_tile[step & 1];
      const bool more = step + 1 < nsteps;
      if (more) fetch(step + 1);

      // ---- 3. S^T = K . Q^T for rows 16w + (0..15) ---------------------------
      f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
      {
        const uint8_t* krow = tb + (wave * kRowsPerWave + n) * kRowStride + 16 * g;
#pragma unroll
        for (int s = 0; s < kDim / 32; ++s) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(krow + 64 * s);
          sacc = mfma_16x16x32(kf, qf[s], sacc);
        }
      }
      // lane (n, g) now holds S[head n][tile row 16w + 4g + j], j = 0..3

      // ---- 4. online softmax ---------------------------------------------------
      const int rbase = step * kTileRows + wave * kRowsPerWave + 4 * g;
      float sv[4];
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sv[j] = (rbase + j < nvalid) ? sacc[j] * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, sv[j]);
      }
      mx = wave_max16(mx);
      if (g == 0) s_red[wave][n] = mx;
      __syncthreads();
      const float mstep = fmaxf(fmaxf(s_red[0][n], s_red[1][n]), fmaxf(s_red[2][n], s_red[3][n]));
      const float m_new = fmaxf(m_run, mstep);  // finite: the tile has a valid row
      const float alpha = exp2f(m_run - m_new);
      float psum = 0.f;
      bf16x4 pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float pj = exp2f(sv[j] - m_new);
        psum += pj;
        pb[j] = static_cast<__bf16>(pj);
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
      *reinterpret_cast<bf16x4*>(&s_p[n * kTileRows + wave * kRowsPerWave + 4 * g]) = pb;
      float aj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) aj[j] = __shfl(alpha, 4 * g + j);
#pragma unroll
      for (int blk = 0; blk < kDBlocks; ++blk)
#pragma unroll
        for (int j = 0; j < 4; ++j) oacc[blk][j] *= aj[j];
      __syncthreads();

      // ---- 5. O[:, 128w .. 128w+127] += P . V ---------------------------------
#pragma unroll
      for (int kk = 0; kk < kTileRows / 32; ++kk) {
        const bf16x8 pf =
            *reinterpret_cast<const bf16x8*>(&s_p[n * kTileRows + 32 * kk + 8 * g]);
        const uint8_t* vb = tb + (32 * kk + 8 * g + (n >> 2)) * kRowStride +
                            (wave * kDPerWave + 4 * (n & 3)) * 2;
#pragma unroll
        for (int blk = 0; blk < kDBlocks; ++blk) {
          const bf16x4 v0 = lds_read_tr16(vb + blk * 32);
          const bf16x4 v1 = lds_read_tr16(vb + 4 * kRowStride + blk * 32);
          const bf16x8 vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          oacc[blk] = mfma_16x16x32(pf, vf, oacc[blk]);
        }
      }
      if (more) stash((step + 1) & 1);
      __syncthreads();
    }
  }

  // ---- 6. epilogue ----------------------------------------------------------
  float lw = wave_sum16(l_run);
  __syncthreads();
  if (g == 0) s_red[wave][n] = lw;
  __syncthreads();
  const float l_tot = s_red[0][n] + s_red[1][n] + s_red[2][n] + s_red[3][n];
  const int dcol = wave * kDPerWave + n;

  if (p.nsplit == 1) {
    const float sink2 = p.sink[n] * kLog2e;
    const float m_tot = fmaxf(m_run, sink2);
    const float a = exp2f(m_run - m_tot);  // 0 when no valid slot
    const float f = a / (a * l_tot + exp2f(sink2 - m_tot));
    float fj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fj[j] = __shfl(f, 4 * g + j);
    __bf16* ob = p.o + bi * p.so_b + mi * p.so_m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      __bf16* orow = ob + int64_t(4 * g + j) * p.so_h + dcol;
#pragma unroll
      for (int blk = 0; blk < kDBlocks; ++blk)
        orow[16 * blk] = static_cast<__bf16>(oacc[blk][j] * fj[j]);
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
        po[(4 * g + j) * kDim + dcol + 16 * blk] = oacc[blk][j];
  }
}

// One work-group per query: thread t owns head t/16, columns 32*(t%16)..+31.
__global__ void __launch_bounds__(256) sa_combine_kernel(const CombineParams p) {
  const int64_t qid = blockIdx.x;
  const int64_t bi = qid / p.m;
  const int64_t mi = qid % p.m;
  const int t = threadIdx.x;
  const int h = t >> 4;
  const int d0 = (t & 15) * 32;
  const float* part = p.part + qid * p.nsplit * kPartFloats;

  float M = -INFINITY;
  for (int s = 0; s < p.nsplit; ++s) M = fmaxf(M, part[s * kPartFloats + h]);
  float L = 0.f;
  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;
  for (int s = 0; s < p.nsplit; ++s) {
    const float* ps = part + s * kPartFloats;
    const float ms = ps[h];
    if (ms == -INFINITY) continue;  // part without a valid slot
    const float w = exp2f(ms - M);
    L += w * ps[kHeads + h];
    const float4* po = reinterpret_cast<const float4*>(ps + 2 * kHeads + h * kDim + d0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = po[i];
      acc[4 * i + 0] += w * v.x;
      acc[4 * i + 1] += w * v.y;
      acc[4 * i + 2] += w * v.z;
      acc[4 * i + 3] += w * v.w;
    }
  }
  const float sink2 = p.sink[h] * kLog2e;
  const float m_tot = fmaxf(M, sink2);
  const float a = exp2f(M - m_tot);
  const float f = a / (a * L + exp2f(sink2 - m_tot));
  __bf16* orow = p.o + bi * p.so_b + mi * p.so_m + int64_t(h) * p.so_h + d0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16x8 v;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = static_cast<__bf16>(acc[8 * i + k] * f);
    *reinterpret_cast<bf16x8*>(orow + 8 * i) = v;
  }
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

}  // namespace

extern "C" {

int sa_abi_version(void) { return SA_ABI_VERSION; }

const char* sa_strerror(int code) {
  switch (code) {
    case SA_OK: return "ok";
    case SA_EINVAL: return "invalid argument (null pointer, size, stride or alignment)";
    case SA_EUNSUPPORTED: return "unsupported shape (needs h == 16, d == 512)";
    case SA_EWORKSPACE: return "workspace missing or too small";
    case SA_EHIP: return "HIP runtime error";
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
  *out_bytes = sa::make_plan(a, cus).ws_bytes;
  return SA_OK;
}

int sa_forward(const sa_args* a, void* hip_stream) {
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  if (a->b == 0 || a->m == 0) return SA_OK;
  int cus = 0;
  const int qrc = current_cus(&cus);
  if (qrc != SA_OK) return qrc;
  const sa::Plan plan = sa::make_plan(a, cus);
  if (plan.ws_bytes > 0 && (a->workspace == nullptr || a->workspace_bytes < plan.ws_bytes))
    return SA_EWORKSPACE;
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);

  FwdParams p{};
  p.q = static_cast<const __bf16*>(a->q);
  p.kv = static_cast<const __bf16*>(a->kv);
  p.sink = a->sink;
  p.idx = a->idx;
  p.o = static_cast<__bf16*>(a->o);
  p.part = static_cast<float*>(a->workspace);
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
  p.scale_log2 = a->scale * kLog2e;
  p.nsplit = plan.nsplit;
  p.split_len = plan.split_len;
  p.nblocks = plan.units * plan.nsplit;

  hipLaunchKernelGGL(sa_fwd_kernel, dim3(unsigned(p.nblocks)), dim3(kThreads), 0, stream, p);
  if (hipGetLastError() != hipSuccess) return SA_EHIP;
  if (plan.nsplit > 1) {
    CombineParams c{};
    c.part = p.part;
    c.sink = a->sink;
    c.o = p.o;
    c.m = a->m;
    c.so_b = a->so[0];
    c.so_m = a->so[1];
    c.so_h = a->so[2];
    c.nsplit = plan.nsplit;
    hipLaunchKernelGGL(sa_combine_kernel, dim3(unsigned(plan.units)), dim3(256), 0, stream, c);
    if (hipGetLastError() != hipSuccess) return SA_EHIP;
  }
  return SA_OK;
}

}  // extern "C"
