// extern "C" surface of libleanstack_amd.so (declared in include/leanstack_amd.h).
//
// Every entry point validates its arguments before touching the GPU, records
// a message for lsk_last_error() on failure and returns a negative status;
// the Python layer turns LSK_ERR_INVALID / LSK_ERR_LAYOUT into ValueError,
// the way src/leanstack/runtime/cutile_logits.py:44-53 rejects bad input
// before launching.

#include "leanstack_amd.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "lsk_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int hip_fail(hipError_t err, const char* what) {
  return fail(LSK_ERR_HIP, "%s: %s (%s)", what, hipGetErrorName(err), hipGetErrorString(err));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

bool packed_layout(int layout_id) {
  return layout_id == LSK_LAYOUT_MFMA16X32 || layout_id == LSK_LAYOUT_MFMA16X32_GATEUP;
}

// Shape rules of the packed layouts: whole 16x32 tiles, and whole gate/up
// row-block pairs for the interleaved layout.
int check_shape(int layout_id, int N, int K) {
  if (!packed_layout(layout_id)) return fail(LSK_ERR_LAYOUT, "unsupported weight layout id %d", layout_id);
  if (N <= 0 || K <= 0) return fail(LSK_ERR_INVALID, "N=%d and K=%d must be positive", N, K);
  if (N % lsk::kTileRows != 0) return fail(LSK_ERR_INVALID, "N=%d must be divisible by %d", N, lsk::kTileRows);
  if (K % lsk::kTileK != 0) return fail(LSK_ERR_INVALID, "K=%d must be divisible by %d", K, lsk::kTileK);
  if (layout_id == LSK_LAYOUT_MFMA16X32_GATEUP && N % (2 * lsk::kTileRows) != 0)
    return fail(LSK_ERR_INVALID, "fused gate_up N=%d must be divisible by %d", N, 2 * lsk::kTileRows);
  return LSK_OK;
}

// Row of the row-major source matrix stored in packed row `pr`.
inline int source_row(int layout_id, int N, int pr) {
  if (layout_id != LSK_LAYOUT_MFMA16X32_GATEUP) return pr;
  const int half = N / 2;
  const int pair = pr / (2 * lsk::kTileRows);
  const int within = pr % (2 * lsk::kTileRows);
  return within < lsk::kTileRows ? pair * lsk::kTileRows + within
                                 : half + pair * lsk::kTileRows + (within - lsk::kTileRows);
}

// Byte offset (in 16-byte units) of W[packed row pr][k8 * 8 .. +8] in the tiles.
inline size_t packed_unit(int K, int pr, int k8) {
  const int KT = K / lsk::kTileK;
  const int rb = pr / lsk::kTileRows;
  const int r = pr % lsk::kTileRows;
  const int kt = k8 / 4;
  const int gq = k8 % 4;
  return ((size_t)rb * KT + kt) * 64 + (size_t)gq * 16 + r;
}

}  // namespace

extern "C" {

int lsk_abi_version(void) { return LSK_ABI_VERSION; }

const char* lsk_last_error(void) { return g_last_error.c_str(); }

size_t lsk_packed_bytes(int layout_id, int N, int K) {
  if (check_shape(layout_id, N, K) != LSK_OK) return 0;
  return (size_t)N * (size_t)K * 2;
}

size_t lsk_workspace_bytes(int op, int M, int N, int K) {
  if (op == LSK_OP_LINEAR) return 0;
  if (op == LSK_OP_LM_HEAD_ARGMAX) {
    if (M < 1 || M > lsk::kDecodeMaxM || N <= 0 || K <= 0 || N % (2 * lsk::kTileRows) != 0) return 0;
    return (size_t)M * (size_t)lsk::lm_head_partials(N) * sizeof(lsk::ArgmaxPartial);
  }
  return 0;
}

int lsk_pack_bf16(const void* w_rowmajor_host, int N, int K, int layout_id, void* out_host) {
  g_last_error.clear();
  if (int st = check_shape(layout_id, N, K)) return st;
  if (w_rowmajor_host == nullptr || out_host == nullptr) return fail(LSK_ERR_INVALID, "null buffer");
  const auto* src = static_cast<const unsigned char*>(w_rowmajor_host);
  auto* dst = static_cast<unsigned char*>(out_host);
  const int k8s = K / 8;
  for (int pr = 0; pr < N; ++pr) {
    const unsigned char* row = src + (size_t)source_row(layout_id, N, pr) * K * 2;
    for (int k8 = 0; k8 < k8s; ++k8) std::memcpy(dst + packed_unit(K, pr, k8) * 16, row + (size_t)k8 * 16, 16);
  }
  return LSK_OK;
}

int lsk_unpack_bf16(const void* packed_host, int N, int K, int layout_id, void* out_rowmajor_host) {
  g_last_error.clear();
  if (int st = check_shape(layout_id, N, K)) return st;
  if (packed_host == nullptr || out_rowmajor_host == nullptr) return fail(LSK_ERR_INVALID, "null buffer");
  const auto* src = static_cast<const unsigned char*>(packed_host);
  auto* dst = static_cast<unsigned char*>(out_rowmajor_host);
  const int k8s = K / 8;
  for (int pr = 0; pr < N; ++pr) {
    unsigned char* row = dst + (size_t)source_row(layout_id, N, pr) * K * 2;
    for (int k8 = 0; k8 < k8s; ++k8) std::memcpy(row + (size_t)k8 * 16, src + packed_unit(K, pr, k8) * 16, 16);
  }
  return LSK_OK;
}

int lsk_linear_bf16(const void* w_packed, int layout_id, int N, int K, const void* x, int M, int ldx, void* y,
                    int ldy, int epilogue, const void* residual, int ldr, void* workspace, size_t ws_bytes,
                    void* hip_stream) {
  (void)workspace;
  (void)ws_bytes;
  g_last_error.clear();
  if (int st = check_shape(layout_id, N, K)) return st;
  if (epilogue != LSK_EPI_NONE && epilogue != LSK_EPI_SILU_MUL && epilogue != LSK_EPI_RESIDUAL_ADD)
    return fail(LSK_ERR_INVALID, "unknown epilogue %d", epilogue);
  if ((epilogue == LSK_EPI_SILU_MUL) != (layout_id == LSK_LAYOUT_MFMA16X32_GATEUP))
    return fail(LSK_ERR_INVALID, "the SiLU*up epilogue requires the interleaved gate_up layout and vice versa");
  if (M < 1) return fail(LSK_ERR_INVALID, "M=%d must be >= 1", M);
  if (w_packed == nullptr || x == nullptr || y == nullptr) return fail(LSK_ERR_INVALID, "null device pointer");
  if (!aligned(w_packed, 16)) return fail(LSK_ERR_INVALID, "packed weights must be 16-byte aligned");
  if (ldx < K || ldx % 8 != 0 || !aligned(x, 16))
    return fail(LSK_ERR_INVALID, "x needs ldx >= K, ldx %% 8 == 0 and 16-byte alignment (ldx=%d, K=%d)", ldx, K);
  const int n_out = epilogue == LSK_EPI_SILU_MUL ? N / 2 : N;
  if (ldy < n_out || ldy % 4 != 0 || !aligned(y, 8))
    return fail(LSK_ERR_INVALID, "y needs ldy >= %d, ldy %% 4 == 0 and 8-byte alignment (ldy=%d)", n_out, ldy);
  if (epilogue == LSK_EPI_RESIDUAL_ADD) {
    if (residual == nullptr || ldr < N || !aligned(residual, 2))
      return fail(LSK_ERR_INVALID, "residual add needs a residual [M][N] with ldr >= N (ldr=%d)", ldr);
  } else if (residual != nullptr) {
    return fail(LSK_ERR_INVALID, "residual given without the residual-add epilogue");
  }
  auto stream = static_cast<hipStream_t>(hip_stream);
  const auto epi = static_cast<lsk::Epilogue>(epilogue);
  hipError_t err;
  const bool gemm_shape = N % lsk::kGemmBN == 0 && K % lsk::kGemmBK == 0;
  if (M <= lsk::kDecodeMaxM) {
    err = lsk::launch_decode_linear(w_packed, N, K, x, M, ldx, y, ldy, epi, residual, ldr, stream);
  } else if (gemm_shape) {
    err = lsk::launch_gemm_linear(w_packed, N, K, x, M, ldx, y, ldy, epi, residual, ldr, stream);
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

int lsk_lm_head_argmax_bf16(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                            float* logits_opt, int logits_mode, long long* out_idx, void* workspace,
                            size_t ws_bytes, void* hip_stream) {
  g_last_error.clear();
  if (layout_id != LSK_LAYOUT_MFMA16X32)
    return fail(LSK_ERR_LAYOUT, "lm_head needs layout %d, got %d", LSK_LAYOUT_MFMA16X32, layout_id);
  if (int st = check_shape(layout_id, V, K)) return st;
  if (V % (2 * lsk::kTileRows) != 0)
    return fail(LSK_ERR_INVALID, "vocab size V=%d must be divisible by %d", V, 2 * lsk::kTileRows);
  if (M < 1 || M > lsk::kDecodeMaxM) return fail(LSK_ERR_INVALID, "M=%d must be in 1..%d", M, lsk::kDecodeMaxM);
  if (logits_mode != LSK_LOGITS_FP32 && logits_mode != LSK_LOGITS_BF16)
    return fail(LSK_ERR_INVALID, "unknown logits mode %d", logits_mode);
  if (w_packed == nullptr || x == nullptr || out_idx == nullptr) return fail(LSK_ERR_INVALID, "null device pointer");
  if (!aligned(w_packed, 16)) return fail(LSK_ERR_INVALID, "packed weights must be 16-byte aligned");
  if (ldx < K || ldx % 8 != 0 || !aligned(x, 16))
    return fail(LSK_ERR_INVALID, "x needs ldx >= K, ldx %% 8 == 0 and 16-byte alignment (ldx=%d, K=%d)", ldx, K);
  if (logits_opt != nullptr && !aligned(logits_opt, 16))
    return fail(LSK_ERR_INVALID, "logits buffer must be 16-byte aligned");
  if (!aligned(out_idx, 8)) return fail(LSK_ERR_INVALID, "out_idx must be 8-byte aligned");
  const size_t need = lsk_workspace_bytes(LSK_OP_LM_HEAD_ARGMAX, M, V, K);
  if (workspace == nullptr || ws_bytes < need || !aligned(workspace, 8))
    return fail(LSK_ERR_WORKSPACE, "lm_head workspace needs %zu bytes, got %zu", need, workspace ? ws_bytes : 0);
  hipError_t err = lsk::launch_lm_head_argmax(w_packed, V, K, x, M, ldx, logits_opt, logits_mode == LSK_LOGITS_BF16,
                                              out_idx, static_cast<lsk::ArgmaxPartial*>(workspace),
                                              static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return hip_fail(err, "lm_head kernel launch");
  return LSK_OK;
}

}  // extern "C"
