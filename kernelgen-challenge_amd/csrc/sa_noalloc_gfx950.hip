// Allocation-free sparse-attention forward: sa_forward_noalloc
// (include/sparse_attn_noalloc.h).
//
// It lives in a library of its own (lib/libsa_noalloc_gfx950.so) because its
// workspace is a file-scope device array that is part of the code object:
// every process that loads this library reserves SA_NOALLOC_SCRATCH_BYTES on
// each GPU it uses, until the process ends. Callers of sa_forward (and the
// torch operators) load only libsparse_attn_gfx950.so and do not carry it.
//
// The entry point runs sa_forward's launches (the kernels live in
// libsparse_attn_gfx950.so) with the workspace pointed at this array. Host
// code never passes `scratch` itself anywhere: on the host the name is only a
// stand-in for the symbol. It uses the device address hipGetSymbolAddress
// returns for the current device, looked up once per device (with that
// device current) on the device's first call.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sa_plan.h"
#include "sparse_attn.h"
#include "sparse_attn_noalloc.h"

namespace {

constexpr int kMaxDevices = 64;
constexpr size_t kScratchBytes = SA_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];
uint8_t* g_scratch[kMaxDevices];  // device address of `scratch`, per device ordinal

int current_scratch(uint8_t** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SA_EHIP;
  uint8_t* p = __atomic_load_n(&g_scratch[dev], __ATOMIC_ACQUIRE);
  if (p == nullptr) {
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr)
      return SA_EHIP;
    p = static_cast<uint8_t*>(addr);
    __atomic_store_n(&g_scratch[dev], p, __ATOMIC_RELEASE);  // a racing thread stores the same
  }
  *out = p;
  return SA_OK;
}

}  // namespace

extern "C" {

int sa_noalloc_scratch_bytes(void) { return int(kScratchBytes); }

int sa_forward_noalloc(const sa_args* a, void* hip_stream) {
  // Host-only checks first (null, shape, strides, flags), as sa_forward
  // makes them; then the workspace size, which needs the device's CU count.
  const int rc = sa::validate(a);
  if (rc != SA_OK) return rc;
  if ((a->flags & SA_FLAG_PLANNED) != 0) return SA_EINVAL;  // a plan lives in a caller's workspace
  if (a->b == 0 || a->m == 0) return SA_OK;
  size_t need = 0;
  const int wrc = sa_workspace_bytes(a, &need);
  if (wrc != SA_OK) return wrc;
  if (need > kScratchBytes) return SA_ESCRATCH;
  uint8_t* ws = nullptr;
  const int src = current_scratch(&ws);
  if (src != SA_OK) return src;
  sa_args b = *a;
  b.workspace = ws;
  b.workspace_bytes = kScratchBytes;
  return sa_forward(&b, hip_stream);
}

}  // extern "C"
