// extern "C" surface of libleanstack_amd.so (declared in include/leanstack_amd.h):
// the entry points that launch kernels or touch device memory.  The packers,
// the argument rules and lsk_last_error() are in host_rules.cpp.
//
// Every entry point validates its arguments before touching the GPU, records
// a message for lsk_last_error() on failure and returns a negative status;
// the Python layer turns LSK_ERR_INVALID / LSK_ERR_LAYOUT into ValueError,
// the way src/leanstack/runtime/cutile_logits.py:44-53 rejects bad input
// before launching.

#include "leanstack_amd.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "lsk_internal.h"

namespace {

using lsk::aligned;
using lsk::check_shape;
using lsk::fail;

int hip_fail(hipError_t err, const char* what) {
  return fail(LSK_ERR_HIP, "%s: %s (%s)", what, hipGetErrorName(err), hipGetErrorString(err));
}

}  // namespace

namespace lsk {
namespace {

// A dispatch timing of one host thread: two events per dispatch, handed out
// in launch order by dispatch_timing_events.
struct DispatchTiming {
  std::vector<hipEvent_t> events;
  int used = 0;
  bool active = false;
};

DispatchTiming& dispatch_timing() {
  thread_local DispatchTiming t;
  return t;
}

void release_events(DispatchTiming& t) {
  for (hipEvent_t e : t.events) (void)hipEventDestroy(e);
  t.events.clear();
  t.used = 0;
  t.active = false;
}

}  // namespace

bool dispatch_timing_events(hipEvent_t* start, hipEvent_t* stop) {
  DispatchTiming& t = dispatch_timing();
  if (!t.active || 2 * (size_t)(t.used + 1) > t.events.size()) return false;
  *start = t.events[2 * t.used];
  *stop = t.events[2 * t.used + 1];
  ++t.used;
  return true;
}

}  // namespace lsk

// Synchronously read and clear word `index` of a workspace.
int read_clear_error_word(void* workspace, int index, int* error_out) {
  if (workspace == nullptr || error_out == nullptr) return fail(LSK_ERR_INVALID, "null argument");
  unsigned word = 0;
  auto* err_word = static_cast<unsigned*>(workspace) + index;
  hipError_t err = hipMemcpy(&word, err_word, sizeof(word), hipMemcpyDeviceToHost);
  if (err != hipSuccess) return hip_fail(err, "hipMemcpy(workspace error word)");
  const unsigned zero = 0;
  err = hipMemcpy(err_word, &zero, sizeof(zero), hipMemcpyHostToDevice);
  if (err != hipSuccess) return hip_fail(err, "hipMemcpy(clear workspace error word)");
  *error_out = (int)word;
  return LSK_OK;
}

extern "C" {

int lsk_abi_version(void) { return LSK_ABI_VERSION; }

size_t lsk_workspace_bytes(int op, int M, int N, int K) {
  if (op == LSK_OP_LINEAR) {
    if (M <= lsk::kDecodeMaxM || N <= 0 || K <= 0) return 0;
    if (M <= lsk::kSkinnyMaxM) {
      // the larger of the plain and the SiLU*up split (lsk_workspace_bytes
      // does not know the epilogue)
      if (!lsk::skinny_route(M, N, K)) return 0;
      int cus = 0;
      if (lsk::current_device_cus(&cus) != hipSuccess) return 0;
      const size_t plain = lsk::skinny_plan(M, N, K, false, cus, true).bytes;
      const size_t silu = N % (2 * lsk::kTileRows) == 0 ? lsk::skinny_plan(M, N, K, true, cus, true).bytes : 0;
      return plain > silu ? plain : silu;
    }
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return 0;
    hipError_t err;
    const size_t bytes = lsk::gemm_workspace_bytes(device, M, N, K, &err);
    return err == hipSuccess ? bytes : 0;
  }
  if (op == LSK_OP_LM_HEAD_ARGMAX) {
    if (M < 1 || M > lsk::kDecodeMaxM || N <= 0 || K <= 0 || N % lsk::kTileRows != 0) return 0;
    return lsk::lm_head_workspace_bytes(M, N);
  }
  return 0;
}

int lsk_linear_plan(int M, int N, int K, size_t ws_bytes, int* plan) {
  lsk::clear_error();
  if (plan == nullptr) return fail(LSK_ERR_INVALID, "plan is NULL");
  if (M < 1 || N < 1 || K < 1) return fail(LSK_ERR_INVALID, "M=%d, N=%d, K=%d must be positive", M, N, K);
  plan[0] = 0;
  plan[1] = 0;
  plan[2] = 0;
  plan[3] = 1;
  // The routing of lsk_linear_bf16: decode kernels up to kDecodeMaxM rows
  // (plan {0, 0, 0, 1}); the skinny kernel where skinny_route takes the
  // shape (plan {weight rows per workgroup, workgroup row groups, groups
  // split, S}, the plain and residual epilogues' plan); the block GEMM on its
  // tile grid; decode slices off it ({0, 0, 0, 1}).
  if (M <= lsk::kDecodeMaxM) return LSK_OK;
  hipError_t err;
  if (lsk::skinny_route(M, N, K)) {
    int cus = 0;
    err = lsk::current_device_cus(&cus);
    if (err != hipSuccess) return hip_fail(err, "device CU count");
    lsk::SkinnyPlan p = lsk::skinny_plan(M, N, K, false, cus, ws_bytes > 0);
    if (p.S > 1 && ws_bytes < p.bytes)
      return fail(LSK_ERR_WORKSPACE, "projection workspace needs %zu bytes (got %zu)", p.bytes, ws_bytes);
    plan[0] = p.rows;
    plan[1] = p.groups;
    plan[2] = p.S > 1 ? p.groups : 0;
    plan[3] = p.S;
    return LSK_OK;
  }
  if (N % lsk::kGemmBN != 0 || K % lsk::kGemmBK != 0) return LSK_OK;
  if (ws_bytes > 0) {
    // The workspace lsk_linear_bf16 would refuse is refused here too.
    int device = 0;
    err = hipGetDevice(&device);
    if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
    const size_t need = lsk::gemm_workspace_bytes(device, M, N, K, &err);
    if (err != hipSuccess) return hip_fail(err, "prefill workspace size");
    if (ws_bytes < need)
      return fail(LSK_ERR_WORKSPACE, "prefill workspace needs %zu bytes (got %zu)", need, ws_bytes);
  }
  err = lsk::plan_gemm_linear(M, N, K, ws_bytes, plan);
  if (err != hipSuccess) return hip_fail(err, "prefill plan");
  return LSK_OK;
}

int lsk_linear_bf16(const void* w_packed, int layout_id, int N, int K, const void* x, int M, int ldx, void* y,
                    int ldy, int epilogue, const void* residual, int ldr, void* workspace, size_t ws_bytes,
                    void* hip_stream) {
  lsk::clear_error();
  if (int st = lsk::check_linear_args(w_packed, layout_id, N, K, x, M, ldx, y, ldy, epilogue, residual, ldr)) return st;
  auto stream = static_cast<hipStream_t>(hip_stream);
  const auto epi = static_cast<lsk::Epilogue>(epilogue);
  hipError_t err;
  const bool gemm_shape = N % lsk::kGemmBN == 0 && K % lsk::kGemmBK == 0;
  if (M <= lsk::kDecodeMaxM) {
    err = lsk::launch_decode_linear(w_packed, N, K, x, M, ldx, y, ldy, epi, residual, ldr, stream);
  } else if (lsk::skinny_route(M, N, K)) {
    int cus = 0;
    err = lsk::current_device_cus(&cus);
    if (err != hipSuccess) return hip_fail(err, "device CU count");
    const lsk::SkinnyPlan p = lsk::skinny_plan(M, N, K, epi == lsk::Epilogue::kSiluMul, cus, workspace != nullptr);
    if (p.S > 1 && (ws_bytes < p.bytes || !aligned(workspace, 256)))
      return fail(LSK_ERR_WORKSPACE, "projection workspace needs %zu bytes, 256-byte aligned (got %zu)", p.bytes,
                  ws_bytes);
    err = lsk::launch_skinny_linear(w_packed, N, K, x, M, ldx, y, ldy, epi, residual, ldr,
                                    p.S > 1 ? workspace : nullptr, ws_bytes, cus, stream);
  } else if (gemm_shape) {
    if (workspace != nullptr) {
      int device = 0;
      err = hipGetDevice(&device);
      if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
      const size_t need = lsk::gemm_workspace_bytes(device, M, N, K, &err);
      if (err != hipSuccess) return hip_fail(err, "prefill workspace size");
      if (ws_bytes < need || !aligned(workspace, 256))
        return fail(LSK_ERR_WORKSPACE, "prefill workspace needs %zu bytes, 256-byte aligned (got %zu)", need, ws_bytes);
    }
    err = lsk::launch_gemm_linear(w_packed, N, K, x, M, ldx, y, ldy, epi, residual, ldr, workspace, ws_bytes,
                                  stream);
  } else {
    // Shapes off the GEMM tile grid: decode kernel over 16-row slices.
    err = hipSuccess;
    for (int m0 = 0; m0 < M && err == hipSuccess; m0 += lsk::kDecodeMaxM) {
      const int mc = M - m0 < lsk::kDecodeMaxM ? M - m0 : lsk::kDecodeMaxM;
      err = lsk::launch_decode_linear(
          w_packed, N, K, static_cast<const __bf16*>(x) + (size_t)m0 * ldx, mc, ldx,
          static_cast<__bf16*>(y) + (size_t)m0 * ldy, ldy, epi,
          residual ? static_cast<const __bf16*>(residual) + (size_t)m0 * ldr : nullptr, ldr, stream);
    }
  }
  if (err != hipSuccess) return hip_fail(err, "projection kernel launch");
  return LSK_OK;
}

int lsk_rmsnorm_linear_bf16(const void* w_packed, int layout_id, int N, int K, const void* x, int M, int ldx,
                            const void* norm_weight, float eps, void* y, int ldy, int epilogue,
                            const void* residual, int ldr, void* hip_stream) {
  lsk::clear_error();
  if (int st = lsk::check_linear_args(w_packed, layout_id, N, K, x, M, ldx, y, ldy, epilogue, residual, ldr)) return st;
  if (M > lsk::kDecodeMaxM)
    return fail(LSK_ERR_INVALID, "the fused RMSNorm projection takes M=1..%d rows (M=%d)", lsk::kDecodeMaxM, M);
  if (norm_weight == nullptr || !aligned(norm_weight, 16))
    return fail(LSK_ERR_INVALID, "the RMSNorm weight [K] must be a 16-byte aligned device pointer");
  if (!std::isfinite(eps) || eps < 0.f) return fail(LSK_ERR_INVALID, "eps=%g must be finite and >= 0", (double)eps);
  hipError_t err = lsk::launch_decode_rmsnorm_linear(w_packed, N, K, x, M, ldx, norm_weight, eps, y, ldy,
                                                     static_cast<lsk::Epilogue>(epilogue), residual, ldr,
                                                     static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "RMSNorm projection kernel launch");
  return LSK_OK;
}

size_t lsk_attention_workspace_bytes(int n_q, int n_kv, int head_dim, int max_seq_len) {
  if (head_dim != lsk::kAttnHeadDim || n_kv < 1 || n_kv > lsk::kAttnMaxKvHeads || n_q < n_kv || n_q % n_kv != 0 ||
      !lsk::attention_group_supported(n_q / n_kv) || max_seq_len < 1 ||
      max_seq_len > lsk::kAttnMaxRows)
    return 0;
  return lsk::attention_workspace_bytes(n_q, n_kv, max_seq_len);
}

namespace {

int check_attention_workspace(int n_q, int n_kv, int max_seq_len, int rows, const void* workspace,
                              size_t ws_bytes) {
  if (rows <= lsk::kAttnMinChunkRows) return LSK_OK;
  const size_t need = lsk::attention_workspace_bytes(n_q, n_kv, max_seq_len);
  if (workspace == nullptr || ws_bytes < need || !aligned(workspace, 256))
    return fail(LSK_ERR_WORKSPACE, "attending up to %d rows needs a workspace of %zu bytes, 256-byte aligned (got %zu)",
                rows, need, workspace ? ws_bytes : 0);
  return LSK_OK;
}

}  // namespace

int lsk_decode_attention_bf16(const void* qkv, int n_q, int n_kv, int head_dim, const void* q_norm_weight,
                              const void* k_norm_weight, float eps, const void* cos, const void* sin, void* k_cache,
                              void* v_cache, int max_seq_len, int pos, float scale, void* out, void* workspace,
                              size_t ws_bytes, void* hip_stream) {
  lsk::clear_error();
  if (int st = lsk::check_attention_args(qkv, n_q, n_kv, head_dim, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache,
                                    v_cache, max_seq_len, scale, out))
    return st;
  if (pos < 0 || pos >= max_seq_len)
    return fail(LSK_ERR_INVALID, "pos=%d, max_seq_len=%d: need 0 <= pos < max_seq_len", pos, max_seq_len);
  if (int st = check_attention_workspace(n_q, n_kv, max_seq_len, pos + 1, workspace, ws_bytes)) return st;
  hipError_t err = lsk::launch_decode_attention(qkv, n_q, n_kv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache,
                                                v_cache, max_seq_len, pos, scale, out, workspace, ws_bytes,
                                                static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "decode attention kernel launch");
  return LSK_OK;
}

int lsk_decode_attention_at_bf16(const void* qkv, int n_q, int n_kv, int head_dim, const void* q_norm_weight,
                                 const void* k_norm_weight, float eps, const void* cos_table, const void* sin_table,
                                 void* k_cache, void* v_cache, int max_seq_len, const int* pos_device, float scale,
                                 void* out, void* workspace, size_t ws_bytes, void* hip_stream) {
  lsk::clear_error();
  if (int st = lsk::check_attention_args(qkv, n_q, n_kv, head_dim, q_norm_weight, k_norm_weight, eps, cos_table,
                                    sin_table, k_cache, v_cache, max_seq_len, scale, out))
    return st;
  if (pos_device == nullptr || !aligned(pos_device, 4))
    return fail(LSK_ERR_INVALID, "pos_device must be a 4-byte aligned device int");
  if (int st = check_attention_workspace(n_q, n_kv, max_seq_len, max_seq_len, workspace, ws_bytes)) return st;
  hipError_t err = lsk::launch_decode_attention_at(qkv, n_q, n_kv, q_norm_weight, k_norm_weight, eps, cos_table,
                                                   sin_table, k_cache, v_cache, max_seq_len, pos_device, scale, out,
                                                   workspace, ws_bytes, static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "decode attention kernel launch");
  return LSK_OK;
}

namespace {

// Checks and launch shared by the plain and the RMSNorm lm_head entry points.
int lm_head_argmax(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                   const void* norm_weight, float eps, float* logits_opt, int logits_mode, long long* out_idx,
                   void* workspace, size_t ws_bytes, void* hip_stream) {
  if (int st = lsk::check_lm_head(w_packed, layout_id, V, K, x, M, ldx, logits_opt, logits_mode, out_idx)) return st;
  const size_t need = lsk_workspace_bytes(LSK_OP_LM_HEAD_ARGMAX, M, V, K);
  if (workspace == nullptr || ws_bytes < need || !aligned(workspace, 8))
    return fail(LSK_ERR_WORKSPACE, "lm_head workspace needs %zu bytes, got %zu", need, workspace ? ws_bytes : 0);
  hipError_t err = lsk::launch_lm_head_argmax(w_packed, V, K, x, M, ldx, logits_opt, logits_mode == LSK_LOGITS_BF16,
                                              out_idx, workspace, norm_weight, eps,
                                              static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "lm_head kernel launch");
  return LSK_OK;
}

}  // namespace

}  // extern "C"

namespace lsk {

int fail_hip_call(hipError_t err, const char* what) { return hip_fail(err, what); }

}  // namespace lsk

extern "C" {

int lsk_lm_head_argmax_bf16(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                            float* logits_opt, int logits_mode, long long* out_idx, void* workspace,
                            size_t ws_bytes, void* hip_stream) {
  lsk::clear_error();
  return lm_head_argmax(w_packed, layout_id, V, K, x, M, ldx, nullptr, 0.f, logits_opt, logits_mode, out_idx,
                        workspace, ws_bytes, hip_stream);
}

int lsk_rmsnorm_lm_head_argmax_bf16(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                                    const void* norm_weight, float eps, float* logits_opt, int logits_mode,
                                    long long* out_idx, void* workspace, size_t ws_bytes, void* hip_stream) {
  lsk::clear_error();
  if (K != 80 * lsk::kTileK || M > 8)
    return fail(LSK_ERR_INVALID, "the RMSNorm lm_head serves K=%d and M <= 8 (got K=%d, M=%d)", 80 * lsk::kTileK, K,
                M);
  if (norm_weight == nullptr || !aligned(norm_weight, 16))
    return fail(LSK_ERR_INVALID, "the norm weight must be a 16-byte aligned device pointer");
  if (!std::isfinite(eps) || eps < 0.f) return fail(LSK_ERR_INVALID, "eps=%g must be finite and >= 0", (double)eps);
  return lm_head_argmax(w_packed, layout_id, V, K, x, M, ldx, norm_weight, eps, logits_opt, logits_mode, out_idx,
                        workspace, ws_bytes, hip_stream);
}

}  // extern "C"

// ----------------------------------------------------------------- stack programs

namespace {

// Persistent grid size per device: CUs x resident workgroups per CU.
int stack_grid(int device, size_t lds_bytes, int* grid_out) {
  static std::mutex mu;
  static std::vector<int> cache;
  std::lock_guard<std::mutex> lock(mu);
  if (device >= (int)cache.size()) cache.resize(device + 1, 0);
  if (cache[device] == 0) {
    int cus = 0;
    hipError_t err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (err != hipSuccess) return hip_fail(err, "hipDeviceGetAttribute(multiprocessor count)");
    int per_cu = 0;
    err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, lsk::stack_kernel_symbol(), lsk::stack_threads(),
                                                       lds_bytes);
    if (err != hipSuccess) return hip_fail(err, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (cus <= 0 || per_cu <= 0) return fail(LSK_ERR_HIP, "stack kernel cannot be resident (cus=%d, per_cu=%d)", cus, per_cu);
    // Every workgroup must be resident at once (they wait for each other).
    const int grid = cus * per_cu;
    cache[device] = grid < lsk::kStackMaxGrid ? grid : lsk::kStackMaxGrid;
  }
  *grid_out = cache[device];
  return LSK_OK;
}

size_t stack_program_bytes(int count) {
  return sizeof(lsk::StackProgram) + (size_t)(count > 1 ? count - 1 : 0) * sizeof(lsk::StackDesc);
}

}  // namespace

extern "C" {

size_t lsk_stack_program_bytes(int count) { return count > 0 ? stack_program_bytes(count) : 0; }

size_t lsk_stack_workspace_bytes(int count) {
  if (count <= 0) return 0;
  int device = 0, grid = 0;
  if (hipGetDevice(&device) != hipSuccess) return 0;
  if (stack_grid(device, lsk::stack_lds_bytes(), &grid) != LSK_OK) return 0;
  return lsk::kStackWsBytes(count, grid);
}

int lsk_stack_prepare(const lsk_projection* projections, int count, int M, void* program_dev, size_t program_bytes) {
  lsk::clear_error();
  if (projections == nullptr || count <= 0) return fail(LSK_ERR_INVALID, "empty stack program");
  if (count > lsk::kStackMaxProjections)
    return fail(LSK_ERR_INVALID, "stack program of %d projections (at most %d)", count, lsk::kStackMaxProjections);
  if (M < 1 || M > lsk::kDecodeMaxM) return fail(LSK_ERR_INVALID, "stack M=%d must be in 1..%d", M, lsk::kDecodeMaxM);
  if (program_dev == nullptr || program_bytes < stack_program_bytes(count) || !aligned(program_dev, 64))
    return fail(LSK_ERR_INVALID, "program buffer needs %zu bytes, 64-byte aligned", stack_program_bytes(count));
  std::vector<unsigned char> host(stack_program_bytes(count), 0);
  auto* prog = reinterpret_cast<lsk::StackProgram*>(host.data());
  prog->count = count;
  prog->M = M;
  prog->magic = lsk::kStackMagic;
  for (int i = 0; i < count; ++i) {
    const lsk_projection& p = projections[i];
    if (int st = check_shape(p.layout_id, p.N, p.K)) {
      const std::string why = lsk::error_message();
      return fail(st, "projection %d: %s", i, why.c_str());
    }
    const int KT = p.K / lsk::kTileK;
    if (KT % lsk::kStackSegTiles != 0)
      return fail(LSK_ERR_INVALID, "projection %d: K=%d must be a multiple of %d", i, p.K,
                  lsk::kStackSegTiles * lsk::kTileK);
    if (p.epilogue != LSK_EPI_NONE && p.epilogue != LSK_EPI_SILU_MUL && p.epilogue != LSK_EPI_RESIDUAL_ADD)
      return fail(LSK_ERR_INVALID, "projection %d: unknown epilogue %d", i, p.epilogue);
    if ((p.epilogue == LSK_EPI_SILU_MUL) != (p.layout_id == LSK_LAYOUT_MFMA16X32_GATEUP))
      return fail(LSK_ERR_INVALID, "projection %d: SiLU*up needs the interleaved gate_up layout and vice versa", i);
    if (p.w_packed == nullptr || p.x == nullptr || p.y == nullptr || !aligned(p.w_packed, 16))
      return fail(LSK_ERR_INVALID, "projection %d: null or misaligned pointer", i);
    if (p.ldx < p.K || p.ldx % 8 != 0 || !aligned(p.x, 16))
      return fail(LSK_ERR_INVALID, "projection %d: x needs ldx >= K, ldx %% 8 == 0, 16-byte alignment", i);
    const int n_out = p.epilogue == LSK_EPI_SILU_MUL ? p.N / 2 : p.N;
    if (p.ldy < n_out || p.ldy % 4 != 0 || !aligned(p.y, 8))
      return fail(LSK_ERR_INVALID, "projection %d: y needs ldy >= %d, ldy %% 4 == 0, 8-byte alignment", i, n_out);
    if (p.epilogue == LSK_EPI_RESIDUAL_ADD) {
      if (p.residual == nullptr || p.ldr < p.N || p.ldr % 4 != 0 || !aligned(p.residual, 8))
        return fail(LSK_ERR_INVALID, "projection %d: residual [M][N] needs ldr >= N, ldr %% 4 == 0, 8-byte alignment",
                    i);
    } else if (p.residual != nullptr) {
      return fail(LSK_ERR_INVALID, "projection %d: residual without the residual-add epilogue", i);
    }
    if (p.depends_on < -1 || p.depends_on >= i)
      return fail(LSK_ERR_INVALID, "projection %d: depends_on=%d must be -1 or an earlier index", i, p.depends_on);
    lsk::StackDesc& d = prog->desc[i];
    d.w = static_cast<const lsk::bf16x8_t*>(p.w_packed);
    d.x = static_cast<const __bf16*>(p.x);
    d.y = static_cast<__bf16*>(p.y);
    d.res = static_cast<const __bf16*>(p.residual);
    d.KT = KT;
    d.ldx = p.ldx;
    d.ldy = p.ldy;
    d.ldr = p.ldr;
    d.epi = p.epilogue;
    d.rbw = p.epilogue == LSK_EPI_SILU_MUL ? 2 : 1;
    d.units = p.N / lsk::kTileRows / d.rbw;
    d.dep = p.depends_on;
  }
  hipError_t err = hipMemcpy(program_dev, host.data(), host.size(), hipMemcpyHostToDevice);
  if (err != hipSuccess) return hip_fail(err, "hipMemcpy(stack program)");
  return LSK_OK;
}

int lsk_stack_run(const void* program_dev, int count, void* workspace, size_t ws_bytes, void* hip_stream) {
  lsk::clear_error();
  if (program_dev == nullptr || count <= 0) return fail(LSK_ERR_INVALID, "null or empty stack program");
  // A workspace below the one-workgroup size is wrong on any device.
  if (workspace == nullptr || ws_bytes < lsk::kStackWsBytes(count, 1) || !aligned(workspace, 256))
    return fail(LSK_ERR_WORKSPACE, "stack workspace needs lsk_stack_workspace_bytes(%d) bytes, 256-byte aligned",
                count);
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  const size_t lds = lsk::stack_lds_bytes();
  int grid = 0;
  if (int st = stack_grid(device, lds, &grid)) return st;
  if (ws_bytes < lsk::kStackWsBytes(count, grid))
    return fail(LSK_ERR_WORKSPACE, "stack workspace needs %zu bytes on this device (got %zu)",
                lsk::kStackWsBytes(count, grid), ws_bytes);
  err = lsk::launch_decode_stack(static_cast<const lsk::StackProgram*>(program_dev), static_cast<unsigned*>(workspace),
                                 grid, lds, static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "stack kernel launch");
  return LSK_OK;
}

int lsk_stack_error(void* workspace, int* error_out) {
  lsk::clear_error();
  return read_clear_error_word(workspace, lsk::kStackWsError, error_out);
}

size_t lsk_probe_workspace_bytes(void) { return lsk::kProbeWsBytes; }

int lsk_probe_stream_step(const void* weights, size_t weight_bytes, const long long* seg_tiles, int count, int mode,
                          int ring, void* workspace, size_t ws_bytes, void* hip_stream) {
  lsk::clear_error();
  if (weights == nullptr || !aligned(weights, 16)) return fail(LSK_ERR_INVALID, "weights must be 16-byte aligned");
  if (seg_tiles == nullptr || count < 1 || count > lsk::kProbeMaxSegments)
    return fail(LSK_ERR_INVALID, "count=%d segments must be in 1..%d", count, lsk::kProbeMaxSegments);
  if (mode < 0 || mode > 3) return fail(LSK_ERR_INVALID, "mode=%d must be 0, 1, 2 or 3", mode);
  if (ring != 4 && ring != 16) return fail(LSK_ERR_INVALID, "ring=%d must be 4 or 16", ring);
  if (workspace == nullptr || ws_bytes < lsk::kProbeWsBytes || !aligned(workspace, 4))
    return fail(LSK_ERR_WORKSPACE, "probe workspace needs %zu bytes (got %zu)", lsk::kProbeWsBytes, ws_bytes);
  int cus = 0;
  hipError_t err = lsk::current_device_cus(&cus);
  if (err != hipSuccess) return hip_fail(err, "device CU count");
  if (mode == 3 && cus > lsk::kProbeMaxTagGroups)
    return fail(LSK_ERR_INVALID, "mode 3 holds tag words for at most %d CUs (the device has %d)",
                lsk::kProbeMaxTagGroups, cus);
  lsk::ProbeSegments seg{};
  seg.count = count;
  unsigned long long total = 0;
  for (int i = 0; i < count; ++i) {
    const long long t = seg_tiles[i];
    if (t <= 0 || t % cus != 0 || t / cus < lsk::kProbeComputeWaves || t / cus > (1 << 30))
      return fail(LSK_ERR_INVALID, "segment %d: %lld tiles must be a multiple of the %d CUs, at least %d per CU", i,
                  t, cus, lsk::kProbeComputeWaves);
    seg.per_cu[i] = (int)(t / cus);
    seg.first[i] = total;
    total += (unsigned long long)t;
  }
  if (total * 1024ull > weight_bytes)
    return fail(LSK_ERR_INVALID, "%llu tiles need %llu weight bytes (got %zu)", total, total * 1024ull, weight_bytes);
  err = lsk::launch_probe_step(weights, seg, mode, ring, cus, workspace, static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "probe kernel launch");
  return LSK_OK;
}

int lsk_probe_mfma_rate(int workgroups, int iterations, void* sink, void* hip_stream) {
  lsk::clear_error();
  if (workgroups < 1 || workgroups > 65536 || iterations < 1 || iterations > (1 << 24))
    return fail(LSK_ERR_INVALID, "workgroups=%d (1..65536) and iterations=%d (1..2^24)", workgroups, iterations);
  if (sink == nullptr || !aligned(sink, 4)) return fail(LSK_ERR_INVALID, "sink must be a 4-byte aligned device word");
  const hipError_t err = lsk::launch_probe_mfma(workgroups, iterations, sink, static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "probe kernel launch");
  return LSK_OK;
}

int lsk_dispatch_timing_begin(int max_dispatches) {
  lsk::DispatchTiming& t = lsk::dispatch_timing();
  if (t.active) return fail(LSK_ERR_INVALID, "a dispatch timing is already active on this thread");
  if (max_dispatches < 1 || max_dispatches > 65536)
    return fail(LSK_ERR_INVALID, "max_dispatches=%d outside 1..65536", max_dispatches);
  t.events.reserve(2 * (size_t)max_dispatches);
  for (int i = 0; i < 2 * max_dispatches; ++i) {
    hipEvent_t e = nullptr;
    const hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      lsk::release_events(t);
      return hip_fail(err, "hipEventCreate");
    }
    t.events.push_back(e);
  }
  t.used = 0;
  t.active = true;
  return LSK_OK;
}

int lsk_dispatch_timing_end(float* durations_us, int capacity, int* dispatches) {
  lsk::DispatchTiming& t = lsk::dispatch_timing();
  if (!t.active) return fail(LSK_ERR_INVALID, "no dispatch timing is active on this thread");
  if (dispatches == nullptr || capacity < 0 || (capacity > 0 && durations_us == nullptr)) {
    lsk::release_events(t);
    return fail(LSK_ERR_INVALID, "null or negative argument");
  }
  for (int i = 0; i < t.used; ++i) {
    float ms = 0.f;
    hipError_t err = hipEventSynchronize(t.events[2 * i + 1]);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, t.events[2 * i], t.events[2 * i + 1]);
    if (err != hipSuccess) {
      lsk::release_events(t);
      return hip_fail(err, "dispatch timing events");
    }
    if (i < capacity) durations_us[i] = ms * 1e3f;
  }
  *dispatches = t.used;
  lsk::release_events(t);
  return LSK_OK;
}

int lsk_linear_error(void* workspace, int* error_out) {
  lsk::clear_error();
  return read_clear_error_word(workspace, 0, error_out);
}

void lsk_set_linear_wait_limit(unsigned polls) { lsk::set_linear_wait_limit(polls); }

}  // extern "C"
