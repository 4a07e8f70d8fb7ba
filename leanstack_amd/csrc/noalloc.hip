// Allocation-free greedy lm_head: lsk_lm_head_argmax_noalloc_bf16.
//
// The same kernel as lsk_lm_head_argmax_bf16 (lm_head_kernel writes one
// (score, index) partial per workgroup and activation row, and its last M
// workgroups reduce them), with its workspace in `scratch`, a file-scope
// device array, instead of a caller-allocated one.  For callers that cannot
// allocate device memory: code under HIP graph capture, tight serving loops.
//
// Limits and sharing: one call's workspace takes 64 + M * P * 8 bytes (P
// scoring workgroups: (V/16 - 512) / 2 + 512 for V/16 > 512, else V/16), at
// most kScratchBytes (1 MiB: every M <= 16 at V = 151936); larger
// calls are rejected before anything touches the GPU.  The array starts
// zeroed (a device global without an initializer) and every call leaves its
// partials zero again, which is the state the kernel needs, so nothing is
// cleared between calls -- but calls that overlap in time on one device
// (unordered streams) race on it.

#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "leanstack_amd.h"
#include "lsk_internal.h"

namespace {

constexpr size_t kScratchBytes = size_t(1) << 20;

// Device code and kernel arguments never name this array from the host: its
// name there is a host-side stand-in, not a device address.  The address
// each device holds it at comes from hipGetSymbolAddress (scratch_address).
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
std::vector<void*> g_scratch_ptr;  // per device id, null until first looked up

// The address of `scratch` on `device` (the current device), looked up
// once per device.
int scratch_address(int device, void** out) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (device >= (int)g_scratch_ptr.size()) g_scratch_ptr.resize(device + 1, nullptr);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return lsk::fail_hip_call(err, "hipGetSymbolAddress(static lm_head scratch)");
    if (ptr == nullptr) return lsk::fail(LSK_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch");
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return LSK_OK;
}

}  // namespace

extern "C" int lsk_lm_head_argmax_noalloc_bf16(const void* w_packed, int layout_id, int V, int K, const void* x,
                                               int M, int ldx, float* logits_opt, int logits_mode,
                                               long long* out_idx, void* hip_stream) {
  if (int st = lsk::check_lm_head_call(w_packed, layout_id, V, K, x, M, ldx, logits_opt, logits_mode, out_idx))
    return st;
  const size_t need = lsk::lm_head_workspace_bytes(M, V);
  if (need > kScratchBytes) {
    return lsk::fail(LSK_ERR_INVALID,
                     "M=%d rows over V=%d need %zu bytes of argmax workspace; the static scratch holds %zu "
                     "(64 + M * P * 8 bytes, P the scoring workgroups): use lsk_lm_head_argmax_bf16 with a workspace",
                     M, V, need, kScratchBytes);
  }
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return lsk::fail_hip_call(err, "hipGetDevice");
  void* workspace = nullptr;
  if (int st = scratch_address(device, &workspace)) return st;
  err = lsk::launch_lm_head_argmax(w_packed, V, K, x, M, ldx, logits_opt, logits_mode == LSK_LOGITS_BF16, out_idx,
                                   workspace, nullptr, 0.f,
                                   static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return lsk::fail_hip_call(err, "lm_head kernel launch");
  return LSK_OK;
}
