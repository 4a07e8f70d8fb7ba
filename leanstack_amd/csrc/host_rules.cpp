// Host-side rules of the C ABI (declared in lsk_host.h): the packers, the
// argument validators and the thread-local message of lsk_last_error().
// Plain C++ with no HIP dependency, so the sanitizer test builds and runs it
// with g++ -fsanitize=address.  The Python layer turns LSK_ERR_INVALID /
// LSK_ERR_LAYOUT into ValueError, the way
// src/leanstack/runtime/cutile_logits.py:44-53 rejects bad input before
// launching.

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "leanstack_amd.h"
#include "lsk_host.h"

namespace lsk {
namespace {

thread_local std::string g_last_error;

bool packed_layout(int layout_id) {
  return layout_id == LSK_LAYOUT_MFMA16X32 || layout_id == LSK_LAYOUT_MFMA16X32_GATEUP;
}

// Row of the row-major source matrix stored in packed row `pr`.
inline int source_row(int layout_id, int N, int pr) {
  if (layout_id != LSK_LAYOUT_MFMA16X32_GATEUP) return pr;
  const int half = N / 2;
  const int pair = pr / (2 * kTileRows);
  const int within = pr % (2 * kTileRows);
  return within < kTileRows ? pair * kTileRows + within : half + pair * kTileRows + (within - kTileRows);
}

// Byte offset (in 16-byte units) of W[packed row pr][k8 * 8 .. +8] in the tiles.
inline size_t packed_unit(int K, int pr, int k8) {
  const int KT = K / kTileK;
  const int rb = pr / kTileRows;
  const int r = pr % kTileRows;
  const int kt = k8 / 4;
  const int gq = k8 % 4;
  return ((size_t)rb * KT + kt) * 64 + (size_t)gq * 16 + r;
}

}  // namespace

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

void clear_error() { g_last_error.clear(); }

const char* error_message() { return g_last_error.c_str(); }

bool attention_group_supported(int group) { return group == 1 || group == 2 || group == 4 || group == 8; }

int check_shape(int layout_id, int N, int K) {
  if (!packed_layout(layout_id)) return fail(LSK_ERR_LAYOUT, "unsupported weight layout id %d", layout_id);
  if (N <= 0 || K <= 0) return fail(LSK_ERR_INVALID, "N=%d and K=%d must be positive", N, K);
  if (N % kTileRows != 0) return fail(LSK_ERR_INVALID, "N=%d must be divisible by %d", N, kTileRows);
  if (K % kTileK != 0) return fail(LSK_ERR_INVALID, "K=%d must be divisible by %d", K, kTileK);
  if (layout_id == LSK_LAYOUT_MFMA16X32_GATEUP && N % (2 * kTileRows) != 0)
    return fail(LSK_ERR_INVALID, "fused gate_up N=%d must be divisible by %d", N, 2 * kTileRows);
  return LSK_OK;
}

int check_linear_args(const void* w_packed, int layout_id, int N, int K, const void* x, int M, int ldx,
                      const void* y, int ldy, int epilogue, const void* residual, int ldr) {
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
  if (ldx > kMaxActivationStride)
    return fail(LSK_ERR_INVALID, "ldx=%d exceeds the largest activation row stride, %d", ldx, kMaxActivationStride);
  const int n_out = epilogue == LSK_EPI_SILU_MUL ? N / 2 : N;
  if (ldy < n_out || ldy % 4 != 0 || !aligned(y, 8))
    return fail(LSK_ERR_INVALID, "y needs ldy >= %d, ldy %% 4 == 0 and 8-byte alignment (ldy=%d)", n_out, ldy);
  if (epilogue == LSK_EPI_RESIDUAL_ADD) {
    if (residual == nullptr || ldr < N || !aligned(residual, 2))
      return fail(LSK_ERR_INVALID, "residual add needs a residual [M][N] with ldr >= N (ldr=%d)", ldr);
  } else if (residual != nullptr) {
    return fail(LSK_ERR_INVALID, "residual given without the residual-add epilogue");
  }
  return LSK_OK;
}

int check_attention_args(const void* qkv, int n_q, int n_kv, int head_dim, const void* q_norm_weight,
                         const void* k_norm_weight, float eps, const void* cos, const void* sin, const void* k_cache,
                         const void* v_cache, int max_seq_len, float scale, const void* out) {
  if (head_dim != kAttnHeadDim)
    return fail(LSK_ERR_INVALID, "head_dim=%d: the attention kernel is built for %d", head_dim, kAttnHeadDim);
  if (n_kv < 1 || n_kv > kAttnMaxKvHeads || n_q < n_kv || n_q % n_kv != 0 || !attention_group_supported(n_q / n_kv))
    return fail(LSK_ERR_INVALID, "n_q=%d, n_kv=%d: n_kv must be 1..%d and n_q 1, 2, 4 or 8 times n_kv", n_q, n_kv,
                kAttnMaxKvHeads);
  if (qkv == nullptr || q_norm_weight == nullptr || k_norm_weight == nullptr || cos == nullptr || sin == nullptr ||
      k_cache == nullptr || v_cache == nullptr || out == nullptr)
    return fail(LSK_ERR_INVALID, "null device pointer");
  if (!aligned(qkv, 2) || !aligned(q_norm_weight, 2) || !aligned(k_norm_weight, 2) || !aligned(cos, 2) ||
      !aligned(sin, 2) || !aligned(out, 2))
    return fail(LSK_ERR_INVALID, "bf16 arguments must be 2-byte aligned");
  if (!aligned(k_cache, 16) || !aligned(v_cache, 16))
    return fail(LSK_ERR_INVALID, "the key and value caches must be 16-byte aligned");
  if (max_seq_len < 1 || max_seq_len > kAttnMaxRows)
    return fail(LSK_ERR_INVALID, "max_seq_len=%d: need 1 <= max_seq_len <= %d", max_seq_len, kAttnMaxRows);
  if (!std::isfinite(eps) || eps < 0.f) return fail(LSK_ERR_INVALID, "eps=%g must be finite and >= 0", (double)eps);
  if (!std::isfinite(scale)) return fail(LSK_ERR_INVALID, "scale must be finite");
  return LSK_OK;
}

int check_lm_head(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                  const float* logits_opt, int logits_mode, const long long* out_idx) {
  if (layout_id != LSK_LAYOUT_MFMA16X32)
    return fail(LSK_ERR_LAYOUT, "lm_head needs layout %d, got %d", LSK_LAYOUT_MFMA16X32, layout_id);
  if (int st = check_shape(layout_id, V, K)) return st;  // V % 16 == 0: whole row-blocks, any count
  if (M < 1 || M > kDecodeMaxM) return fail(LSK_ERR_INVALID, "M=%d must be in 1..%d", M, kDecodeMaxM);
  if (logits_mode != LSK_LOGITS_FP32 && logits_mode != LSK_LOGITS_BF16)
    return fail(LSK_ERR_INVALID, "unknown logits mode %d", logits_mode);
  if (w_packed == nullptr || x == nullptr || out_idx == nullptr) return fail(LSK_ERR_INVALID, "null device pointer");
  if (!aligned(w_packed, 16)) return fail(LSK_ERR_INVALID, "packed weights must be 16-byte aligned");
  if (ldx < K || ldx % 8 != 0 || !aligned(x, 16))
    return fail(LSK_ERR_INVALID, "x needs ldx >= K, ldx %% 8 == 0 and 16-byte alignment (ldx=%d, K=%d)", ldx, K);
  if (logits_opt != nullptr && !aligned(logits_opt, 16))
    return fail(LSK_ERR_INVALID, "logits buffer must be 16-byte aligned");
  if (!aligned(out_idx, 8)) return fail(LSK_ERR_INVALID, "out_idx must be 8-byte aligned");
  return LSK_OK;
}

int check_lm_head_call(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                       const float* logits_opt, int logits_mode, const long long* out_idx) {
  clear_error();
  return check_lm_head(w_packed, layout_id, V, K, x, M, ldx, logits_opt, logits_mode, out_idx);
}

}  // namespace lsk

extern "C" {

const char* lsk_last_error(void) { return lsk::error_message(); }

size_t lsk_packed_bytes(int layout_id, int N, int K) {
  if (lsk::check_shape(layout_id, N, K) != LSK_OK) return 0;
  return (size_t)N * (size_t)K * 2;
}

int lsk_pack_bf16(const void* w_rowmajor_host, int N, int K, int layout_id, void* out_host) {
  lsk::clear_error();
  if (int st = lsk::check_shape(layout_id, N, K)) return st;
  if (w_rowmajor_host == nullptr || out_host == nullptr) return lsk::fail(LSK_ERR_INVALID, "null buffer");
  const auto* src = static_cast<const unsigned char*>(w_rowmajor_host);
  auto* dst = static_cast<unsigned char*>(out_host);
  const int k8s = K / 8;
  for (int pr = 0; pr < N; ++pr) {
    const unsigned char* row = src + (size_t)lsk::source_row(layout_id, N, pr) * K * 2;
    for (int k8 = 0; k8 < k8s; ++k8) std::memcpy(dst + lsk::packed_unit(K, pr, k8) * 16, row + (size_t)k8 * 16, 16);
  }
  return LSK_OK;
}

int lsk_unpack_bf16(const void* packed_host, int N, int K, int layout_id, void* out_rowmajor_host) {
  lsk::clear_error();
  if (int st = lsk::check_shape(layout_id, N, K)) return st;
  if (packed_host == nullptr || out_rowmajor_host == nullptr) return lsk::fail(LSK_ERR_INVALID, "null buffer");
  const auto* src = static_cast<const unsigned char*>(packed_host);
  auto* dst = static_cast<unsigned char*>(out_rowmajor_host);
  const int k8s = K / 8;
  for (int pr = 0; pr < N; ++pr) {
    unsigned char* row = dst + (size_t)lsk::source_row(layout_id, N, pr) * K * 2;
    for (int k8 = 0; k8 < k8s; ++k8) std::memcpy(row + (size_t)k8 * 16, src + lsk::packed_unit(K, pr, k8) * 16, 16);
  }
  return LSK_OK;
}

}  // extern "C"
