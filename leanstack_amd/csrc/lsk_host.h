// Host-side rules of the C ABI that need no HIP: tile geometry, the packed
// layouts' index arithmetic, argument validation and the thread-local error
// message of lsk_last_error().  Defined in host_rules.cpp, which builds with a
// plain C++ compiler (the sanitizer test builds it with g++
// -fsanitize=address).  Not part of the ABI.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "leanstack_amd.h"

namespace lsk {

// Tile geometry of LSK_LAYOUT_MFMA16X32: 16 rows x 32 K of bf16 = 1024 bytes,
// one v_mfma_f32_16x16x32_bf16 operand per 64-lane wavefront.
constexpr int kTileRows = 16;
constexpr int kTileK = 32;
constexpr int kTileBytes = kTileRows * kTileK * 2;

// Largest M served by the decode/verify kernel (the MFMA column count).
constexpr int kDecodeMaxM = 16;

// Largest activation row stride (elements) of a projection: the prefill
// kernel reads a 256-row block of x through a buffer descriptor whose byte
// offsets are 32-bit, so 256 * ldx * 2 must stay below 2^31 (and ldx is a
// multiple of 8).
constexpr int kMaxActivationStride = (1 << 22) - 8;

// Decode attention geometry (attention.hip): up to kAttnMinChunkRows rows
// attended run as one chunk (one workgroup per kv head, no combine); up to
// 8 * kAttnSplitRows rows as at most 8 chunks of kAttnSplitRows rows (one
// combine round); beyond that, at most kAttnMaxChunks chunks of the smallest
// multiple of kAttnMinChunkRows rows that allows it.
constexpr int kAttnHeadDim = 128;
constexpr int kAttnMinChunkRows = 128;
constexpr int kAttnSplitRows = 64;
constexpr int kAttnMaxChunkRows = 512;
constexpr int kAttnMaxChunks = 32;
constexpr int kAttnMaxRows = kAttnMaxChunks * kAttnMaxChunkRows;  // 16384
constexpr int kAttnMaxKvHeads = 64;
static_assert(kAttnSplitRows % 16 == 0 && kAttnSplitRows >= 16 && kAttnSplitRows <= kAttnMinChunkRows,
              "chunks are whole 16-row MFMA groups, at most one workgroup's 128");

// Rows per chunk when `rows` rows (1..kAttnMaxRows) are attended; the host
// and the kernel share it.
constexpr int attention_rows_per_chunk(int rows) {
  if (rows <= kAttnMinChunkRows) return kAttnMinChunkRows;
  if (rows <= 8 * kAttnSplitRows) return kAttnSplitRows;
  const int units = (rows + kAttnMinChunkRows - 1) / kAttnMinChunkRows;
  return kAttnMinChunkRows * ((units + kAttnMaxChunks - 1) / kAttnMaxChunks);
}

// Chunk slots per kv head that a position below max_seq_len can need.
constexpr int attention_most_chunks(int max_seq_len) {
  if (max_seq_len <= kAttnMinChunkRows) return 1;
  if (max_seq_len <= 8 * kAttnSplitRows) return (max_seq_len + kAttnSplitRows - 1) / kAttnSplitRows;
  const int units = (max_seq_len + kAttnMinChunkRows - 1) / kAttnMinChunkRows;
  const int most = units > 8 ? units : 8;
  return most < kAttnMaxChunks ? most : kAttnMaxChunks;
}

// Record `fmt` as this thread's lsk_last_error() message; returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char* error_message();

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// q heads per kv head the attention kernel is built for.
bool attention_group_supported(int group);

// Shape rules of the packed layouts (whole 16x32 tiles, whole gate/up pairs).
int check_shape(int layout_id, int N, int K);

// Argument rules of the projection entry points (see lsk_linear_bf16).
int check_linear_args(const void* w_packed, int layout_id, int N, int K, const void* x, int M, int ldx,
                      const void* y, int ldy, int epilogue, const void* residual, int ldr);

// Argument rules shared by both decode attention entry points (all but pos
// and the workspace).
int check_attention_args(const void* qkv, int n_q, int n_kv, int head_dim, const void* q_norm_weight,
                         const void* k_norm_weight, float eps, const void* cos, const void* sin, const void* k_cache,
                         const void* v_cache, int max_seq_len, float scale, const void* out);

// Every lm_head argument rule but the workspace's.
int check_lm_head(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                  const float* logits_opt, int logits_mode, const long long* out_idx);

// check_lm_head after clearing the error message (for entry points defined
// outside abi.cpp).
int check_lm_head_call(const void* w_packed, int layout_id, int V, int K, const void* x, int M, int ldx,
                       const float* logits_opt, int logits_mode, const long long* out_idx);

}  // namespace lsk
