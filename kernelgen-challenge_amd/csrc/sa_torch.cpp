// sa_torch.cpp -- thin PyTorch-ROCm operator over the sparse_attn C-ABI.
//
// Registers torch.ops.sa_amd.sparse_attn_fwd. It checks devices and dtypes,
// allocates the output (like track-01/submission.py:1000) and the split-topk
// workspace through the caching allocator, and calls sa_forward on the
// current HIP stream. No kernel code lives here.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "sparse_attn.h"

namespace {

at::Tensor sparse_attn_fwd(const at::Tensor& q, const at::Tensor& kv,
                           const at::Tensor& attn_sink,
                           const at::Tensor& topk_idxs, double scale,
                           const c10::optional<at::Tensor>& err, int64_t flags) {
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
  const at::Tensor sink_c = attn_sink.contiguous();
  at::Tensor o = at::empty({b, m, h, d}, q.options());

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
  TORCH_CHECK_VALUE(flags >= 0 && flags <= 0xFFFFFFFFll, "bad flags ", flags);
  a.flags = static_cast<uint32_t>(flags);
  if (err.has_value()) {
    TORCH_CHECK(err->device() == q.device() && err->scalar_type() == at::kInt &&
                    err->numel() >= 1 && err->is_contiguous(),
                "err must be a contiguous int32 tensor on q's device");
    a.err_word = err->data_ptr<int32_t>();
  }

  size_t ws = 0;
  int rc = sa_workspace_bytes(&a, &ws);
  TORCH_CHECK_VALUE(rc != SA_EINVAL && rc != SA_EUNSUPPORTED,
                    "sparse_attn: ", sa_strerror(rc));
  TORCH_CHECK(rc == SA_OK, "sparse_attn: ", sa_strerror(rc));
  at::Tensor workspace;
  if (ws > 0) {
    workspace = at::empty({static_cast<int64_t>(ws)}, q.options().dtype(at::kByte));
    a.workspace = workspace.data_ptr();
    a.workspace_bytes = ws;
  }
  rc = sa_forward(&a, c10::hip::getCurrentHIPStream().stream());
  TORCH_CHECK_VALUE(rc != SA_EINVAL && rc != SA_EUNSUPPORTED,
                    "sparse_attn: ", sa_strerror(rc));
  TORCH_CHECK(rc == SA_OK, "sparse_attn: ", sa_strerror(rc));
  return o;
}

}  // namespace

TORCH_LIBRARY(sa_amd, m) {
  m.def(
      "sparse_attn_fwd(Tensor q, Tensor kv, Tensor attn_sink, Tensor topk_idxs, "
      "float scale, Tensor? err=None, int flags=0) -> Tensor");
}

TORCH_LIBRARY_IMPL(sa_amd, CUDA, m) { m.impl("sparse_attn_fwd", &sparse_attn_fwd); }
