// Internal declarations shared by the C-ABI layer (abi.cpp) and the gfx950
// kernel translation units (decode.hip, gemm.hip).  Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lsk {

// Tile geometry of LSK_LAYOUT_MFMA16X32: 16 rows x 32 K of bf16 = 1024 bytes,
// one v_mfma_f32_16x16x32_bf16 operand per 64-lane wavefront.
constexpr int kTileRows = 16;
constexpr int kTileK = 32;
constexpr int kTileBytes = kTileRows * kTileK * 2;

// Largest M served by the decode/verify kernel (the MFMA column count).
constexpr int kDecodeMaxM = 16;

// Prefill GEMM block tile: BN weight rows x BM tokens x BK.
constexpr int kGemmBN = 128;
constexpr int kGemmBM = 128;
constexpr int kGemmBK = 64;

// Argmax partial written by each lm_head workgroup: (score, index).
struct ArgmaxPartial {
  float score;
  int index;
};

enum class Epilogue : int { kNone = 0, kSiluMul = 1, kResidualAdd = 2 };

// Decode / verify launch (M <= 16).  All pointers are device pointers that
// the caller has validated.  Returns the hipError_t of the launch.
hipError_t launch_decode_linear(const void* w, int N, int K, const void* x, int M, int ldx,
                                void* y, int ldy, Epilogue epi, const void* residual, int ldr,
                                hipStream_t stream);

// Number of workgroups (= argmax partials per row) the lm_head kernel uses.
int lm_head_partials(int V);

hipError_t launch_lm_head_argmax(const void* w, int V, int K, const void* x, int M, int ldx,
                                 float* logits, int logits_bf16, long long* out_idx,
                                 ArgmaxPartial* partials, hipStream_t stream);

// Prefill GEMM launch (any M >= 1; used for M > kDecodeMaxM).
hipError_t launch_gemm_linear(const void* w, int N, int K, const void* x, int M, int ldx,
                              void* y, int ldy, Epilogue epi, const void* residual, int ldr,
                              hipStream_t stream);

}  // namespace lsk
