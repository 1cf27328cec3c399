// ssa_bwd_noalloc: the backward of ssa_bwd for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).  No reference counterpart.
//
// ssa_bwd needs two caller workspaces: Delta ([B, Hq, N] fp32) and the dn/db
// partials (2 * B * Hkv * ceil(N / 128) fp32).  Here both live in `scratch`,
// a file-scope device array of SSA_NOALLOC_SCRATCH_BYTES bytes that every
// device the library runs on holds until the process ends.  The host never
// passes the array's name to a kernel (in host code it is a stand-in, not a
// device address): on the first call on a device, with that device current,
// hipGetSymbolAddress gives that device's copy, and the address is kept per
// device.  dQ takes the recompute path (no dS' workspace).
//
// Contents persist between calls.  Nothing needs clearing: the preprocess
// writes every Delta row before dK/dV and dQ read it, and every dK/dV
// workgroup (including those that exit early) writes its own partial before
// the reduction reads it.  Calls on one device share the array, so two calls
// in flight at once on one device (on different streams) race.
#include <mutex>

#include "../../include/ssa_mi355x.h"
#include "ssa_launch.hpp"

namespace {

static __device__ __align__(256) char scratch[SSA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // per device: the address of `scratch` there

// Address of the current device's copy of `scratch`, looked up once per device.
int32_t scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SSA_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return SSA_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SSA_OK;
}

int64_t round256(int64_t x) { return (x + 255) & ~static_cast<int64_t>(255); }

}  // namespace

extern "C" int32_t ssa_bwd_noalloc(const ssa_bwd_args* a, void* stream) {
  if (a == nullptr) return SSA_ERR_NULL_POINTER;
  // Validated like ssa_bwd; the caller's delta, partials and ds_workspace
  // fields are ignored.
  ssa::BwdParams p{};
  const int32_t st = ssa::fill_bwd_params(a, &p, false, false, false);
  if (st != SSA_OK) return st;
  const int64_t delta_bytes = round256(static_cast<int64_t>(a->batch) * a->heads_q * a->seqlen * 4);
  const int64_t part_bytes = 2ll * a->batch * a->heads_kv * ssa::dkdv_key_blocks(a->seqlen) * 4;
  if (delta_bytes + part_bytes > SSA_NOALLOC_SCRATCH_BYTES) return SSA_ERR_SCRATCH;
  void* base = nullptr;
  const int32_t sst = scratch_of_current_device(&base);
  if (sst != SSA_OK) return sst;
  p.delta = static_cast<float*>(base);
  p.partials = reinterpret_cast<float*>(static_cast<char*>(base) + delta_bytes);
  p.ds = nullptr;
  return ssa::run_bwd(p, a->dtype, a->head_dim, a->causal != 0, static_cast<hipStream_t>(stream));
}
