// sa_torch.cpp -- thin PyTorch-ROCm operators over the C-ABIs of this package.
//
// Registers torch.ops.sa_amd.sparse_attn_fwd (o), sparse_attn_fwd_lse
// (o, lse), sparse_attn_merge (o, lse of merged partials), sparse_attn_plan
// (the index plan of a topk_idxs tensor) and the planned forwards
// sparse_attn_fwd_planned / sparse_attn_fwd_lse_planned, the track-02
// operator hc_split_sinkhorn (pre, post, comb) over include/hc_sinkhorn.h and
// the track-03 operator fused_moe over include/fused_moe.h.
// They check devices and dtypes, allocate the outputs (like
// track-01/submission.py:1000 and track-02/submission.py:353-355) and the
// workspace through the caching allocator, and call the C-ABIs on the
// current HIP stream. No kernel code lives here.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/csrc/utils/pybind.h>
#include <torch/library.h>

#include <mutex>

#include "fused_moe.h"
#include "hc_sinkhorn.h"
#include "sparse_attn.h"

namespace {

void check_rc(int rc, const char* what) {
  TORCH_CHECK_VALUE(rc != SA_EINVAL && rc != SA_EUNSUPPORTED, what, ": ", sa_strerror(rc));
  TORCH_CHECK(rc == SA_OK, what, ": ", sa_strerror(rc));
}

// Deferred index check: one int32 per device in mapped pinned host memory,
// passed to the kernels as sa_args.err_word. A kernel that meets an index
// outside [-1, kv_len) stores 1 into it; the host reads it with a plain load,
// so a call never waits for the GPU to learn of an earlier call's bad index.
// Allocated on first use and kept until the process ends.
constexpr int kMaxFlagDevices = 64;
struct HostFlag {
  int32_t* host = nullptr;  // host address (read / cleared by Python)
  int32_t* dev = nullptr;   // the same word as the GPU addresses it
};
std::mutex g_flag_mu;
HostFlag g_flags[kMaxFlagDevices];

HostFlag host_flag(int device) {
  TORCH_CHECK(device >= 0 && device < kMaxFlagDevices, "device index ", device, " out of range");
  std::lock_guard<std::mutex> lock(g_flag_mu);
  HostFlag& f = g_flags[device];
  if (f.host == nullptr) {
    const c10::DeviceGuard guard(c10::Device(c10::DeviceType::CUDA, device));
    void* h = nullptr;
    TORCH_CHECK(hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocPortable) == hipSuccess,
                "sparse_attn: hipHostMalloc of the index-error flag failed");
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
      (void)hipHostFree(h);
      TORCH_CHECK(false, "sparse_attn: hipHostGetDevicePointer of the index-error flag failed");
    }
    *static_cast<volatile int32_t*>(h) = 0;
    f.host = static_cast<int32_t*>(h);
    f.dev = static_cast<int32_t*>(d);
  }
  return f;
}

// Host address of the device's deferred index-error flag (an int32).
int64_t index_error_flag_address(int64_t device) {
  return static_cast<int64_t>(reinterpret_cast<uintptr_t>(host_flag(int(device)).host));
}

// err_word of a call: the caller's device tensor, else the deferred flag when
// asked for, else none.
int32_t* err_word(const c10::optional<at::Tensor>& err, bool deferred_check,
                  const at::Device& dev) {
  if (err.has_value()) {
    TORCH_CHECK(err->device() == dev && err->scalar_type() == at::kInt &&
                    err->numel() >= 1 && err->is_contiguous(),
                "err must be a contiguous int32 tensor on q's device");
    return err->data_ptr<int32_t>();
  }
  return deferred_check ? host_flag(dev.index()).dev : nullptr;
}

// o, and lse when `want_lse` (fp32 [b, m, h]).
// `plan`: the workspace of sparse_attn_plan for these indices (the forward
// then skips the index kernels), or none.
std::tuple<at::Tensor, at::Tensor> forward(const at::Tensor& q, const at::Tensor& kv,
                                           const at::Tensor& attn_sink,
                                           const at::Tensor& topk_idxs, double scale,
                                           const c10::optional<at::Tensor>& err,
                                           int64_t flags, bool deferred_check, bool want_lse,
                                           const c10::optional<at::Tensor>& plan) {
  TORCH_CHECK_VALUE(q.dim() == 4, "q must be [b, m, h, d], got ", q.sizes());
  TORCH_CHECK_VALUE(kv.dim() == 3, "kv must be [b, kv_len, d], got ", kv.sizes());
  TORCH_CHECK_VALUE(attn_sink.dim() == 1, "attn_sink must be [h], got ",
                    attn_sink.sizes());
  TORCH_CHECK_VALUE(topk_idxs.dim() == 3, "topk_idxs must be [b, m, topk], got ",
                    topk_idxs.sizes());
  TORCH_CHECK_TYPE(q.scalar_type() == at::kBFloat16, "q must be bfloat16");
  TORCH_CHECK_TYPE(kv.scalar_type() == at::kBFloat16, "kv must be bfloat16");
  TORCH_CHECK_TYPE(attn_sink.scalar_type() == at::kFloat, "attn_sink must be float32");
  TORCH_CHECK_TYPE(topk_idxs.scalar_type() == at::kInt, "topk_idxs must be int32");
  TORCH_CHECK(q.is_cuda() && kv.device() == q.device() &&
                  attn_sink.device() == q.device() && topk_idxs.device() == q.device(),
              "all inputs must be on the same GPU");
  const int64_t b = q.size(0), m = q.size(1), h = q.size(2), d = q.size(3);
  TORCH_CHECK_VALUE(kv.size(0) == b && kv.size(2) == d, "kv shape ", kv.sizes(),
                    " does not match q ", q.sizes());
  TORCH_CHECK_VALUE(attn_sink.size(0) == h, "attn_sink must have h entries");
  TORCH_CHECK_VALUE(topk_idxs.size(0) == b && topk_idxs.size(1) == m,
                    "topk_idxs shape ", topk_idxs.sizes(), " does not match q ",
                    q.sizes());

  const c10::DeviceGuard guard(q.device());
  const at::Tensor sink_c = attn_sink.is_contiguous() ? attn_sink : attn_sink.contiguous();
  at::Tensor o = at::empty({b, m, h, d}, q.options());
  at::Tensor lse;

  sa_args a{};
  a.q = q.data_ptr();
  a.kv = kv.data_ptr();
  a.sink = sink_c.data_ptr<float>();
  a.idx = topk_idxs.data_ptr<int32_t>();
  a.o = o.data_ptr();
  a.b = b;
  a.m = m;
  a.h = h;
  a.d = d;
  a.kv_len = kv.size(1);
  a.topk = topk_idxs.size(2);
  for (int i = 0; i < 4; ++i) a.sq[i] = q.stride(i);
  for (int i = 0; i < 3; ++i) a.skv[i] = kv.stride(i);
  for (int i = 0; i < 3; ++i) a.sidx[i] = topk_idxs.stride(i);
  for (int i = 0; i < 4; ++i) a.so[i] = o.stride(i);
  a.scale = static_cast<float>(scale);
  TORCH_CHECK_VALUE(flags >= 0 && flags <= 0xFFFFFFFFll && (flags & SA_FLAG_PLANNED) == 0,
                    "bad flags ", flags);
  a.flags = static_cast<uint32_t>(flags);
  a.err_word = err_word(err, deferred_check, q.device());
  if (want_lse) {
    lse = at::empty({b, m, h}, q.options().dtype(at::kFloat));
    a.lse = lse.data_ptr<float>();
    for (int i = 0; i < 3; ++i) a.slse[i] = lse.stride(i);
  }

  size_t ws = 0;
  check_rc(sa_workspace_bytes(&a, &ws), "sparse_attn");
  at::Tensor workspace;
  if (plan.has_value()) {
    TORCH_CHECK_VALUE(plan->scalar_type() == at::kByte && plan->dim() == 1 &&
                          plan->is_contiguous() && plan->device() == q.device() &&
                          static_cast<size_t>(plan->numel()) >= ws,
                      "plan is not an index plan of these arguments");
    a.workspace = ws > 0 ? plan->data_ptr() : nullptr;
    a.workspace_bytes = ws;
    a.flags |= SA_FLAG_PLANNED;
  } else if (ws > 0) {
    workspace = at::empty({static_cast<int64_t>(ws)}, q.options().dtype(at::kByte));
    a.workspace = workspace.data_ptr();
    a.workspace_bytes = ws;
  }
  check_rc(sa_forward(&a, c10::hip::getCurrentHIPStream().stream()), "sparse_attn");
  return {o, lse};
}

// The index plan of (q's shape, kv's length and row stride, topk_idxs): a
// byte tensor holding the workspace that sa_plan_indices fills. q and kv are
// read for their shapes and strides only.
at::Tensor sparse_attn_plan(const at::Tensor& q, const at::Tensor& kv,
                            const at::Tensor& topk_idxs, const c10::optional<at::Tensor>& err,
                            int64_t flags, bool deferred_check) {
  TORCH_CHECK_VALUE(q.dim() == 4 && kv.dim() == 3 && topk_idxs.dim() == 3,
                    "expected q [b, m, h, d], kv [b, kv_len, d], topk_idxs [b, m, topk]");
  TORCH_CHECK_TYPE(q.scalar_type() == at::kBFloat16 && kv.scalar_type() == at::kBFloat16,
                   "q and kv must be bfloat16");
  TORCH_CHECK_TYPE(topk_idxs.scalar_type() == at::kInt, "topk_idxs must be int32");
  TORCH_CHECK(q.is_cuda() && kv.device() == q.device() && topk_idxs.device() == q.device(),
              "all inputs must be on the same GPU");
  TORCH_CHECK_VALUE(kv.size(0) == q.size(0) && topk_idxs.size(0) == q.size(0) &&
                        topk_idxs.size(1) == q.size(1),
                    "shapes of q ", q.sizes(), ", kv ", kv.sizes(), ", topk_idxs ",
                    topk_idxs.sizes(), " do not match");
  TORCH_CHECK_VALUE(flags >= 0 && flags <= 0xFFFFFFFFll && (flags & SA_FLAG_PLANNED) == 0,
                    "bad flags ", flags);
  const c10::DeviceGuard guard(q.device());
  sa_args a{};
  a.q = q.data_ptr();
  a.kv = kv.data_ptr();
  a.sink = static_cast<const float*>(q.data_ptr());  // not read by the index kernels
  a.idx = topk_idxs.data_ptr<int32_t>();
  a.o = q.data_ptr();                                 // not written by the index kernels
  a.b = q.size(0);
  a.m = q.size(1);
  a.h = q.size(2);
  a.d = q.size(3);
  a.kv_len = kv.size(1);
  a.topk = topk_idxs.size(2);
  for (int i = 0; i < 4; ++i) a.sq[i] = q.stride(i);
  for (int i = 0; i < 3; ++i) a.skv[i] = kv.stride(i);
  for (int i = 0; i < 3; ++i) a.sidx[i] = topk_idxs.stride(i);
  for (int i = 0; i < 4; ++i) a.so[i] = q.stride(i);
  a.scale = 1.f;
  a.flags = static_cast<uint32_t>(flags);
  a.err_word = err_word(err, deferred_check, q.device());
  size_t ws = 0;
  check_rc(sa_workspace_bytes(&a, &ws), "sparse_attn_plan");
  at::Tensor workspace = at::empty({static_cast<int64_t>(ws)}, q.options().dtype(at::kByte));
  a.workspace = ws > 0 ? workspace.data_ptr() : nullptr;
  a.workspace_bytes = ws;
  check_rc(sa_plan_indices(&a, c10::hip::getCurrentHIPStream().stream()), "sparse_attn_plan");
  return workspace;
}

at::Tensor sparse_attn_fwd(const at::Tensor& q, const at::Tensor& kv,
                           const at::Tensor& attn_sink, const at::Tensor& topk_idxs,
                           double scale, const c10::optional<at::Tensor>& err, int64_t flags,
                           bool deferred_check) {
  return std::get<0>(
      forward(q, kv, attn_sink, topk_idxs, scale, err, flags, deferred_check, false, {}));
}

at::Tensor sparse_attn_fwd_planned(const at::Tensor& q, const at::Tensor& kv,
                                   const at::Tensor& attn_sink, const at::Tensor& topk_idxs,
                                   double scale, const at::Tensor& plan,
                                   const c10::optional<at::Tensor>& err, int64_t flags,
                                   bool deferred_check) {
  return std::get<0>(
      forward(q, kv, attn_sink, topk_idxs, scale, err, flags, deferred_check, false, plan));
}

std::tuple<at::Tensor, at::Tensor> sparse_attn_fwd_lse(
    const at::Tensor& q, const at::Tensor& kv, const at::Tensor& attn_sink,
    const at::Tensor& topk_idxs, double scale, const c10::optional<at::Tensor>& err,
    int64_t flags, bool deferred_check) {
  return forward(q, kv, attn_sink, topk_idxs, scale, err, flags, deferred_check, true, {});
}

std::tuple<at::Tensor, at::Tensor> sparse_attn_fwd_lse_planned(
    const at::Tensor& q, const at::Tensor& kv, const at::Tensor& attn_sink,
    const at::Tensor& topk_idxs, double scale, const at::Tensor& plan,
    const c10::optional<at::Tensor>& err, int64_t flags, bool deferred_check) {
  return forward(q, kv, attn_sink, topk_idxs, scale, err, flags, deferred_check, true, plan);
}

// Merge n partials: o_parts bf16 [n, b, m, h, d], lse_parts fp32 [n, b, m, h].
std::tuple<at::Tensor, at::Tensor> sparse_attn_merge(const at::Tensor& o_parts,
                                                     const at::Tensor& lse_parts,
                                                     const c10::optional<at::Tensor>& sink) {
  TORCH_CHECK_VALUE(o_parts.dim() == 5, "o_parts must be [n, b, m, h, d], got ",
                    o_parts.sizes());
  TORCH_CHECK_VALUE(lse_parts.dim() == 4, "lse_parts must be [n, b, m, h], got ",
                    lse_parts.sizes());
  TORCH_CHECK_TYPE(o_parts.scalar_type() == at::kBFloat16, "o_parts must be bfloat16");
  TORCH_CHECK_TYPE(lse_parts.scalar_type() == at::kFloat, "lse_parts must be float32");
  TORCH_CHECK(o_parts.is_cuda() && lse_parts.device() == o_parts.device(),
              "o_parts and lse_parts must be on the same GPU");
  const int64_t n = o_parts.size(0), b = o_parts.size(1), m = o_parts.size(2),
                h = o_parts.size(3), d = o_parts.size(4);
  TORCH_CHECK_VALUE(lse_parts.size(0) == n && lse_parts.size(1) == b &&
                        lse_parts.size(2) == m && lse_parts.size(3) == h,
                    "lse_parts shape ", lse_parts.sizes(), " does not match o_parts ",
                    o_parts.sizes());
  const c10::DeviceGuard guard(o_parts.device());
  const at::Tensor op = o_parts.contiguous();
  const at::Tensor lp = lse_parts.contiguous();
  at::Tensor sink_c;
  if (sink.has_value()) {
    TORCH_CHECK_TYPE(sink->scalar_type() == at::kFloat, "attn_sink must be float32");
    TORCH_CHECK_VALUE(sink->dim() == 1 && sink->size(0) == h, "attn_sink must be [h]");
    TORCH_CHECK(sink->device() == o_parts.device(), "attn_sink must be on the same GPU");
    sink_c = sink->contiguous();
  }
  at::Tensor o = at::empty({b, m, h, d}, o_parts.options());
  at::Tensor lse = at::empty({b, m, h}, o_parts.options().dtype(at::kFloat));
  sa_merge_args a{};
  a.o_parts = op.data_ptr();
  a.lse_parts = lp.data_ptr<float>();
  a.sink = sink.has_value() ? sink_c.data_ptr<float>() : nullptr;
  a.o = o.data_ptr();
  a.lse = lse.data_ptr<float>();
  a.n = n;
  a.b = b;
  a.m = m;
  a.h = h;
  a.d = d;
  for (int i = 0; i < 5; ++i) a.sop[i] = op.stride(i);
  for (int i = 0; i < 4; ++i) a.slp[i] = lp.stride(i);
  for (int i = 0; i < 4; ++i) a.so[i] = o.stride(i);
  for (int i = 0; i < 3; ++i) a.slse[i] = lse.stride(i);
  check_rc(sa_merge(&a, c10::hip::getCurrentHIPStream().stream()), "sparse_attn_merge");
  return {o, lse};
}

// track-02: mixes fp32 [b, s, 24], hc_scale fp32 [3], hc_base fp32 [24].
// Returns pre [b, s, 4], post [b, s, 4], comb [b, s, 4, 4] (fp32).
std::tuple<at::Tensor, at::Tensor, at::Tensor> hc_split_sinkhorn_op(
    const at::Tensor& mixes, const at::Tensor& hc_scale, const at::Tensor& hc_base,
    int64_t hc_mult, int64_t sinkhorn_iters, double eps, int64_t flags) {
  TORCH_CHECK_VALUE(mixes.dim() == 3, "mixes must be 3-D [b, s, 24], got ", mixes.sizes());
  TORCH_CHECK_VALUE(hc_mult == 4, "hc_split_sinkhorn is built for hc_mult = 4, got ", hc_mult);
  TORCH_CHECK_VALUE(mixes.size(2) == 24, "mixes last dim must be 24, got ", mixes.size(2));
  TORCH_CHECK_VALUE(hc_scale.numel() == 3 && hc_base.numel() == 24,
                    "hc_scale must have 3 and hc_base 24 elements");
  for (const at::Tensor* t : {&mixes, &hc_scale, &hc_base})
    TORCH_CHECK_TYPE(t->scalar_type() == at::kFloat, "mixes, hc_scale and hc_base must be float32");
  TORCH_CHECK(mixes.is_cuda() && hc_scale.device() == mixes.device() &&
                  hc_base.device() == mixes.device(),
              "mixes, hc_scale and hc_base must be on the same GPU");
  TORCH_CHECK_VALUE(sinkhorn_iters >= INT32_MIN && sinkhorn_iters <= INT32_MAX,
                    "sinkhorn_iters out of range");
  const c10::DeviceGuard guard(mixes.device());
  // (each tensor op below goes through the dispatcher: a small call's host
  // time is mostly these, so inputs that are already fine are not touched)
  at::Tensor x = mixes.is_contiguous() ? mixes : mixes.contiguous();
  if ((reinterpret_cast<uintptr_t>(x.data_ptr()) & 15u) != 0) x = x.clone();  // 16-byte rows
  const at::Tensor sc = hc_scale.is_contiguous() ? hc_scale : hc_scale.contiguous();
  const at::Tensor bs = hc_base.is_contiguous() ? hc_base : hc_base.contiguous();
  const int64_t b = mixes.size(0), s = mixes.size(1), n = b * s;
  // One allocation, three contiguous outputs carved from it (pre, post, comb)
  at::Tensor out = at::empty({24 * n}, x.options());
  at::Tensor pre = out.as_strided({b, s, 4}, {4 * s, 4, 1}, 0);
  at::Tensor post = out.as_strided({b, s, 4}, {4 * s, 4, 1}, 4 * n);
  at::Tensor comb = out.as_strided({b, s, 4, 4}, {16 * s, 16, 4, 1}, 8 * n);
  hc_args a{};
  a.mixes = x.data_ptr<float>();
  a.scale = sc.data_ptr<float>();
  a.base = bs.data_ptr<float>();
  a.pre = pre.data_ptr<float>();
  a.post = post.data_ptr<float>();
  a.comb = comb.data_ptr<float>();
  a.n = n;
  a.hc_mult = int32_t(hc_mult);
  a.iters = int32_t(sinkhorn_iters);
  a.eps = float(eps);
  a.flags = uint32_t(flags);
  const int rc = hc_split_sinkhorn(&a, c10::hip::getCurrentHIPStream().stream());
  TORCH_CHECK_VALUE(rc != HC_EINVAL && rc != HC_EUNSUPPORTED, "hc_split_sinkhorn: ",
                    hc_strerror(rc));
  TORCH_CHECK(rc == HC_OK, "hc_split_sinkhorn: ", hc_strerror(rc));
  return {pre, post, comb};
}

// track-03: hidden bf16 [M, K], w1 bf16 [E, 2N, K], w2 bf16 [E, K, N],
// score bf16 [M, E]. Returns out bf16 [M, K] (track-03/submission.py:293-294
// allocates it the same way).
at::Tensor fused_moe_op(const at::Tensor& hidden, const at::Tensor& w1, const at::Tensor& w2,
                        const at::Tensor& score, int64_t topk, bool renormalize,
                        int64_t flags) {
  TORCH_CHECK_VALUE(hidden.dim() == 2 && w1.dim() == 3 && w2.dim() == 3 && score.dim() == 2,
                    "expected hidden [M, K], w1 [E, 2N, K], w2 [E, K, N], score [M, E]");
  for (const at::Tensor* t : {&hidden, &w1, &w2, &score})
    TORCH_CHECK_TYPE(t->scalar_type() == at::kBFloat16,
                     "fused_moe: hidden, w1, w2 and score must be bfloat16");
  TORCH_CHECK(hidden.is_cuda() && w1.device() == hidden.device() &&
                  w2.device() == hidden.device() && score.device() == hidden.device(),
              "fused_moe: all inputs must be on the same GPU");
  const int64_t M = hidden.size(0), K = hidden.size(1), E = w1.size(0), N = w2.size(2);
  TORCH_CHECK_VALUE(w1.size(1) == 2 * N && w1.size(2) == K && w2.size(0) == E &&
                        w2.size(1) == K && score.size(0) == M && score.size(1) == E,
                    "fused_moe: shapes hidden ", hidden.sizes(), ", w1 ", w1.sizes(), ", w2 ",
                    w2.sizes(), ", score ", score.sizes(), " do not match");
  TORCH_CHECK_VALUE(flags >= 0 && flags <= 0xFFFFFFFFll, "bad flags ", flags);
  const c10::DeviceGuard guard(hidden.device());
  const at::Tensor h = hidden.contiguous(), a1 = w1.contiguous(), a2 = w2.contiguous(),
                   sc = score.contiguous();
  at::Tensor out = at::empty({M, K}, hidden.options());
  fm_args a{};
  a.hidden = h.data_ptr();
  a.w1 = a1.data_ptr();
  a.w2 = a2.data_ptr();
  a.score = sc.data_ptr();
  a.out = out.data_ptr();
  a.M = M;
  a.K = K;
  a.N = N;
  a.E = E;
  a.topk = topk;
  a.s_hidden = K;
  a.s_score = E;
  a.s_out = K;
  a.renormalize = renormalize ? 1 : 0;
  a.flags = static_cast<uint32_t>(flags);
  size_t ws = 0;
  auto rc_check = [](int rc) {
    TORCH_CHECK_VALUE(rc != FM_EINVAL && rc != FM_EUNSUPPORTED, "fused_moe: ", fm_strerror(rc));
    TORCH_CHECK(rc == FM_OK, "fused_moe: ", fm_strerror(rc));
  };
  rc_check(fm_workspace_bytes(&a, &ws));
  at::Tensor workspace;
  if (ws > 0) {
    workspace = at::empty({static_cast<int64_t>(ws)}, hidden.options().dtype(at::kByte));
    a.workspace = workspace.data_ptr();
    a.workspace_bytes = ws;
  }
  rc_check(fm_forward(&a, c10::hip::getCurrentHIPStream().stream()));
  return out;
}

}  // namespace

TORCH_LIBRARY(sa_amd, m) {
  // deferred_check: with err = None, report bad indices into the device's
  // mapped host flag (index_error_flag_address) instead of nowhere.
  m.def(
      "sparse_attn_fwd(Tensor q, Tensor kv, Tensor attn_sink, Tensor topk_idxs, "
      "float scale, Tensor? err=None, int flags=0, bool deferred_check=False) -> Tensor");
  m.def(
      "sparse_attn_fwd_lse(Tensor q, Tensor kv, Tensor attn_sink, Tensor topk_idxs, "
      "float scale, Tensor? err=None, int flags=0, bool deferred_check=False) -> (Tensor, Tensor)");
  m.def("sparse_attn_merge(Tensor o_parts, Tensor lse_parts, Tensor? attn_sink=None) -> "
        "(Tensor, Tensor)");
  m.def(
      "sparse_attn_plan(Tensor q, Tensor kv, Tensor topk_idxs, Tensor? err=None, int flags=0, "
      "bool deferred_check=False) -> Tensor");
  m.def(
      "sparse_attn_fwd_planned(Tensor q, Tensor kv, Tensor attn_sink, Tensor topk_idxs, "
      "float scale, Tensor plan, Tensor? err=None, int flags=0, bool deferred_check=False) "
      "-> Tensor");
  m.def(
      "sparse_attn_fwd_lse_planned(Tensor q, Tensor kv, Tensor attn_sink, Tensor topk_idxs, "
      "float scale, Tensor plan, Tensor? err=None, int flags=0, bool deferred_check=False) "
      "-> (Tensor, Tensor)");
  m.def(
      "hc_split_sinkhorn(Tensor mixes, Tensor hc_scale, Tensor hc_base, int hc_mult=4, "
      "int sinkhorn_iters=20, float eps=1e-6, int flags=0) -> (Tensor, Tensor, Tensor)");
  m.def("index_error_flag_address(int device) -> int");
  m.def(
      "fused_moe(Tensor hidden, Tensor w1, Tensor w2, Tensor score, int topk, "
      "bool renormalize=False, int flags=0) -> Tensor");
}

TORCH_LIBRARY_IMPL(sa_amd, CUDA, m) {
  m.impl("sparse_attn_fwd", &sparse_attn_fwd);
  m.impl("sparse_attn_fwd_lse", &sparse_attn_fwd_lse);
  m.impl("sparse_attn_merge", &sparse_attn_merge);
  m.impl("sparse_attn_plan", &sparse_attn_plan);
  m.impl("sparse_attn_fwd_planned", &sparse_attn_fwd_planned);
  m.impl("sparse_attn_fwd_lse_planned", &sparse_attn_fwd_lse_planned);
  m.impl("hc_split_sinkhorn", &hc_split_sinkhorn_op);
  m.impl("fused_moe", &fused_moe_op);
}

// No tensor argument: registered for every dispatch key.
TORCH_LIBRARY_IMPL(sa_amd, CatchAll, m) {
  m.impl("index_error_flag_address", &index_error_flag_address);
}

// The same operators as plain Python functions of this module (sa_torch_ext),
// for the drop-ins: a call through torch.ops boxes every argument and result
// for the dispatcher, which costs several microseconds, more than the whole
// kernel of a small call. torch.ops.sa_amd.* stays registered for callers
// that need the dispatcher. Argument names and defaults follow the schemas
// above.
PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  namespace py = pybind11;
  using py::arg;
  m.def("sparse_attn_fwd", &sparse_attn_fwd, arg("q"), arg("kv"), arg("attn_sink"),
        arg("topk_idxs"), arg("scale"), arg("err") = py::none(), arg("flags") = 0,
        arg("deferred_check") = false);
  m.def("sparse_attn_fwd_lse", &sparse_attn_fwd_lse, arg("q"), arg("kv"), arg("attn_sink"),
        arg("topk_idxs"), arg("scale"), arg("err") = py::none(), arg("flags") = 0,
        arg("deferred_check") = false);
  m.def("sparse_attn_fwd_planned", &sparse_attn_fwd_planned, arg("q"), arg("kv"),
        arg("attn_sink"), arg("topk_idxs"), arg("scale"), arg("plan"), arg("err") = py::none(),
        arg("flags") = 0, arg("deferred_check") = false);
  m.def("sparse_attn_fwd_lse_planned", &sparse_attn_fwd_lse_planned, arg("q"), arg("kv"),
        arg("attn_sink"), arg("topk_idxs"), arg("scale"), arg("plan"), arg("err") = py::none(),
        arg("flags") = 0, arg("deferred_check") = false);
  m.def("hc_split_sinkhorn", &hc_split_sinkhorn_op, arg("mixes"), arg("hc_scale"),
        arg("hc_base"), arg("hc_mult") = 4, arg("sinkhorn_iters") = 20, arg("eps") = 1e-6,
        arg("flags") = 0);
  m.def("fused_moe", &fused_moe_op, arg("hidden"), arg("w1"), arg("w2"), arg("score"),
        arg("topk"), arg("renormalize") = false, arg("flags") = 0);
}
