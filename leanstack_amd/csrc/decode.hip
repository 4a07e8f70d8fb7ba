// Decode (M = 1) and speculative-verify (M = 2..16) projections for gfx950.
//
// The weights are HBM-bound: every byte of W is read exactly once per call and
// the arithmetic intensity is M FLOP/byte.  The kernel therefore streams the
// packed 1 KB tiles (LSK_LAYOUT_MFMA16X32) with one 16-byte load per lane and
// feeds each tile straight into v_mfma_f32_16x16x32_bf16 as the A operand.
// The activations x[M][K] form the B operand, padded with zero columns up to
// 16, so M = 1..16 all cost the same HBM bytes and the same instruction
// count: the verify batch rides along with the decode step for free.
//
// Work split: one workgroup owns RBW row-blocks (16 output rows each) and its
// NW wavefronts split the K tiles; partial 16x16 fp32 tiles are summed
// through LDS in wave order, so results are bitwise reproducible.
//
// Reference arithmetic replaced: torch.mv / F.linear at
// src/leanstack/runtime/qwen_explicit.py:787, :913, :942, :948 (M = 1) and
// :748, :819, :828, :830 (verify M = 2..k+1), plus the SiLU(gate)*up of
// :829-830 / :943-948, the residual adds of :820 / :831 / :949, and the
// lm_head argmax of src/leanstack/runtime/cutile_logits.py:17-31, :67-69 and
// qwen_explicit.py:952-960.

#include <hip/hip_runtime.h>

#include <climits>

#include "lsk_internal.h"

namespace lsk {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Weights are touched once per step; keep them out of the caches' way.
__device__ __forceinline__ bf16x8_t load_weight_tile(const bf16x8_t* p) {
  return __builtin_nontemporal_load(p);
}

// Activation fragment of one K tile.  Padding lanes (m >= M) read row 0,
// which is always in bounds, and clear it with a bit mask instead of a
// branch, so the load stays unconditional.
__device__ __forceinline__ bf16x8_t load_x_frag(const bf16x8_t* p, unsigned keep) {
  u32x4_t v = __builtin_bit_cast(u32x4_t, *p);
  v &= keep;
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ unsigned short bf16_bits(float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}

__device__ __forceinline__ float bf16_round(float v) {
  return static_cast<float>(static_cast<__bf16>(v));
}

__device__ __forceinline__ float bf16_to_f32(__bf16 v) { return static_cast<float>(v); }

// SiLU(g) * u with the rounding chain of the reference: the gate_up product is
// a bf16 tensor, F.silu returns bf16, and the product is rounded to bf16
// (src/leanstack/runtime/qwen_explicit.py:828-830, :942-948).
__device__ __forceinline__ float silu_mul_bf16(float g_acc, float u_acc) {
  const float g = bf16_round(g_acc);
  const float u = bf16_round(u_acc);
  const float s = bf16_round(g / (1.0f + expf(-g)));
  return bf16_round(s * u);
}

// Accumulate RBW row-blocks over this wave's K range into acc.
//   wt   : tile (rb0, 0) of the workgroup, already offset by `lane`
//   xrow : x row (m, or row 0 for padding lanes), as 16-byte units, + g
// U > 0: the range is exactly U k-tiles and every weight load of the wave is
// issued in one round (one memory latency per wave).  U == 0: any length,
// in rounds of 8 / RBW k-tiles plus a remainder.
template <int RBW, int U>
__device__ __forceinline__ void accumulate_rows(f32x4_t (&acc)[RBW], const bf16x8_t* __restrict__ wt,
                                                const bf16x8_t* __restrict__ xrow, bool m_active,
                                                int KT, int kb, int ke) {
  const unsigned keep = m_active ? 0xffffffffu : 0u;
  if constexpr (U > 0) {
    // One round: every weight load of the wave goes out first (the HBM
    // latency is paid once), then the activation fragments -- L2 hits --
    // are fetched next to the multiplies that use them, which keeps the
    // register footprint at the weights plus a short window.
    bf16x8_t wv[U][RBW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int r = 0; r < RBW; ++r) wv[u][r] = load_weight_tile(wt + ((size_t)r * KT + kb + u) * 64);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bf16x8_t xv = load_x_frag(xrow + (kb + u) * 4, keep);
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xv, acc[r]);
    }
    (void)ke;
  } else {
    constexpr int R = 8 / RBW;
    int kt = kb;
    for (; kt + R <= ke; kt += R) {
      bf16x8_t xv[R];
      bf16x8_t wv[R][RBW];
#pragma unroll
      for (int u = 0; u < R; ++u) {
        xv[u] = load_x_frag(xrow + (kt + u) * 4, keep);
#pragma unroll
        for (int r = 0; r < RBW; ++r) wv[u][r] = load_weight_tile(wt + ((size_t)r * KT + kt + u) * 64);
      }
#pragma unroll
      for (int u = 0; u < R; ++u) {
#pragma unroll
        for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xv[u], acc[r]);
      }
    }
    for (; kt < ke; ++kt) {
      const bf16x8_t xv = load_x_frag(xrow + kt * 4, keep);
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(load_weight_tile(wt + ((size_t)r * KT + kt) * 64), xv, acc[r]);
    }
  }
}

// Sum the NW per-wave partial tiles in wave order into wave 0's acc.
// Returns false on every wave other than 0 (those are done).
template <int NW, int RBW>
__device__ __forceinline__ bool reduce_waves(f32x4_t (&acc)[RBW], int wave, int lane) {
  if constexpr (NW == 1) {
    return true;
  } else {
    __shared__ f32x4_t red[NW - 1][RBW][64];
    if (wave > 0) {
#pragma unroll
      for (int r = 0; r < RBW; ++r) red[wave - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave != 0) return false;
#pragma unroll
    for (int w = 0; w < NW - 1; ++w) {
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] += red[w][r][lane];
    }
    return true;
  }
}

// y = epilogue(x . W^T) for M <= 16.  Grid: (NB / RBW) workgroups of NW waves;
// U > 0 requires K/32 == NW * U (single-round loads).
template <int NW, int RBW, int EPI, int U>
__global__ __launch_bounds__(NW * 64) void decode_linear_kernel(
    const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x, int ldx, __bf16* __restrict__ y,
    int ldy, const __bf16* __restrict__ residual, int ldr, int M, int KT) {
  static_assert(EPI != static_cast<int>(Epilogue::kSiluMul) || RBW == 2,
                "SiLU*up pairs one gate and one up row-block per workgroup");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = lane & 15;  // B-operand column = activation row
  const int g = lane >> 4;  // K group inside a tile / output row quad
  const bool m_active = m < M;
  const int rb0 = blockIdx.x * RBW;
  const int kb = (KT * wave) / NW;
  const int ke = (KT * (wave + 1)) / NW;

  f32x4_t acc[RBW];
#pragma unroll
  for (int r = 0; r < RBW; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const bf16x8_t* xrow = reinterpret_cast<const bf16x8_t*>(x + (size_t)(m_active ? m : 0) * ldx) + g;
  const bf16x8_t* wt = w + (size_t)rb0 * KT * 64 + lane;
  accumulate_rows<RBW, U>(acc, wt, xrow, m_active, KT, kb, ke);

  if (!reduce_waves<NW, RBW>(acc, wave, lane)) return;
  if (!m_active) return;

  // Lane (g, m) holds output rows 4g..4g+3 of each row-block for column m.
  if constexpr (EPI == static_cast<int>(Epilogue::kSiluMul)) {
    const int j = blockIdx.x * 16 + 4 * g;  // intermediate index
    unsigned short o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = bf16_bits(silu_mul_bf16(acc[0][i], acc[1][i]));
    *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + j) =
        u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
  } else {
#pragma unroll
    for (int r = 0; r < RBW; ++r) {
      const int n = (rb0 + r) * 16 + 4 * g;
      unsigned short o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = bf16_round(acc[r][i]);
        if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd))
          v = bf16_to_f32(residual[(size_t)m * ldr + n + i]) + v;
        o[i] = bf16_bits(v);
      }
      *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + n) =
          u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
    }
  }
}

// lm_head scores for RBW row-blocks (vocab rows) + the workgroup's argmax.
// Grid: (NB / RBW) workgroups; partial[m * P + blockIdx.x] = best (score, index).
template <int NW, int RBW, int U>
__global__ __launch_bounds__(NW * 64) void lm_head_kernel(
    const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x, int ldx, float* __restrict__ logits,
    int V, int logits_bf16, ArgmaxPartial* __restrict__ partial, int M, int KT) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = lane & 15;
  const int g = lane >> 4;
  const bool m_active = m < M;
  const int rb0 = blockIdx.x * RBW;
  const int kb = (KT * wave) / NW;
  const int ke = (KT * (wave + 1)) / NW;

  f32x4_t acc[RBW];
#pragma unroll
  for (int r = 0; r < RBW; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bf16x8_t* xrow = reinterpret_cast<const bf16x8_t*>(x + (size_t)(m_active ? m : 0) * ldx) + g;
  const bf16x8_t* wt = w + (size_t)rb0 * KT * 64 + lane;
  accumulate_rows<RBW, U>(acc, wt, xrow, m_active, KT, kb, ke);

  if (!reduce_waves<NW, RBW>(acc, wave, lane)) return;

  // Scan this lane's rows in increasing index order: strict '>' keeps the
  // lowest index among equal scores, the torch.argmax convention.
  float best = -__builtin_huge_valf();
  int best_idx = INT_MAX;
#pragma unroll
  for (int r = 0; r < RBW; ++r) {
    const int n0 = (rb0 + r) * 16 + 4 * g;
    f32x4_t s = acc[r];
    if (logits_bf16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = bf16_round(s[i]);
    }
    if (logits != nullptr && m_active) *reinterpret_cast<f32x4_t*>(logits + (size_t)m * V + n0) = s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (s[i] > best) {
        best = s[i];
        best_idx = n0 + i;
      }
    }
  }
  // Lanes m, m+16, m+32, m+48 hold the same column: combine them.
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float os = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_idx, off);
    if (os > best || (os == best && oi < best_idx)) {
      best = os;
      best_idx = oi;
    }
  }
  if (g == 0 && m_active) partial[(size_t)m * gridDim.x + blockIdx.x] = ArgmaxPartial{best, best_idx};
}

// Second stage: one workgroup per activation row reduces the P partials,
// as the host-side torch.argmax over tile maxima does in
// src/leanstack/runtime/cutile_logits.py:67-69.  Each thread issues all of
// its partial loads before comparing, so the stage costs about one memory
// latency.
constexpr int kFinalizeThreads = 1024;
constexpr int kFinalizePerThread = 8;

__device__ __forceinline__ void better_of(float& best, int& best_idx, float s, int i) {
  if (s > best || (s == best && i < best_idx)) {
    best = s;
    best_idx = i;
  }
}

__global__ __launch_bounds__(kFinalizeThreads) void argmax_finalize_kernel(const ArgmaxPartial* __restrict__ partial,
                                                                           int P, long long* __restrict__ out_idx) {
  const int m = blockIdx.x;
  const ArgmaxPartial* row = partial + (size_t)m * P;
  float best = -__builtin_huge_valf();
  int best_idx = INT_MAX;
  for (int base = 0; base < P; base += kFinalizeThreads * kFinalizePerThread) {
    ArgmaxPartial c[kFinalizePerThread];
#pragma unroll
    for (int j = 0; j < kFinalizePerThread; ++j) {
      const int p = base + j * kFinalizeThreads + (int)threadIdx.x;
      c[j] = p < P ? row[p] : ArgmaxPartial{-__builtin_huge_valf(), INT_MAX};
    }
#pragma unroll
    for (int j = 0; j < kFinalizePerThread; ++j) better_of(best, best_idx, c[j].score, c[j].index);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float os = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_idx, off);
    better_of(best, best_idx, os, oi);
  }
  constexpr int kW = kFinalizeThreads / 64;
  __shared__ float s_best[kW];
  __shared__ int s_idx[kW];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_best[wave] = best;
    s_idx[wave] = best_idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kW; ++w) better_of(best, best_idx, s_best[w], s_idx[w]);
    out_idx[m] = best_idx;
  }
}

constexpr int kLmHeadWaves = 8;
constexpr int kLmHeadRBW = 2;

template <int NW, int RBW, int EPI, int U>
hipError_t launch_decode_cfg(const void* w, int NB, int KT, const void* x, int M, int ldx, void* y,
                             int ldy, const void* residual, int ldr, hipStream_t stream) {
  decode_linear_kernel<NW, RBW, EPI, U><<<dim3(NB / RBW), dim3(NW * 64), 0, stream>>>(
      static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, static_cast<__bf16*>(y), ldy,
      static_cast<const __bf16*>(residual), ldr, M, KT);
  return hipGetLastError();
}

// Shape dispatch: the Qwen3-4B K values get single-round instantiations
// (K/32 = 80 -> 16 waves x 5 for QKV and the gate/up pairs, 128 -> 8 x 16,
// 304 -> 16 x 19, each measured faster than the alternatives on MI355X); any
// other K runs the round-based variant.
template <int RBW, int EPI>
hipError_t launch_decode_shape(const void* w, int NB, int KT, const void* x, int M, int ldx, void* y, int ldy,
                               const void* residual, int ldr, hipStream_t stream) {
  switch (KT) {
    case 80:
      // 16 waves x 5 k-tiles, for the single row-block (QKV) and the gate/up
      // pair alike: measured 4.5 % / 3.2 % faster than 8 waves x 10 (whose
      // gate/up form needs 96 VGPRs and leaves 96 of 608 workgroups for a
      // second wave) and than the round-based loop.
      return launch_decode_cfg<16, RBW, EPI, 5>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
    case 128:
      if constexpr (RBW == 1) return launch_decode_cfg<8, RBW, EPI, 16>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
      break;
    case 304:
      if constexpr (RBW == 1) return launch_decode_cfg<16, RBW, EPI, 19>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
      break;
    default:
      break;
  }
  if (KT >= 256) return launch_decode_cfg<16, RBW, EPI, 0>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
  return launch_decode_cfg<8, RBW, EPI, 0>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
}

}  // namespace

hipError_t launch_decode_linear(const void* w, int N, int K, const void* x, int M, int ldx, void* y,
                                int ldy, Epilogue epi, const void* residual, int ldr, hipStream_t stream) {
  const int NB = N / kTileRows;
  const int KT = K / kTileK;
  switch (epi) {
    case Epilogue::kSiluMul:
      return launch_decode_shape<2, 1>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
    case Epilogue::kResidualAdd:
      return launch_decode_shape<1, 2>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
    case Epilogue::kNone:
    default:
      return launch_decode_shape<1, 0>(w, NB, KT, x, M, ldx, y, ldy, residual, ldr, stream);
  }
}

int lm_head_partials(int V) { return (V / kTileRows) / kLmHeadRBW; }

hipError_t launch_lm_head_argmax(const void* w, int V, int K, const void* x, int M, int ldx, float* logits,
                                 int logits_bf16, long long* out_idx, ArgmaxPartial* partials,
                                 hipStream_t stream) {
  const int NB = V / kTileRows;
  const int KT = K / kTileK;
  const int P = NB / kLmHeadRBW;
  if (KT == 80) {
    lm_head_kernel<kLmHeadWaves, kLmHeadRBW, 10><<<dim3(P), dim3(kLmHeadWaves * 64), 0, stream>>>(
        static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, logits, V, logits_bf16, partials, M,
        KT);
  } else {
    lm_head_kernel<kLmHeadWaves, kLmHeadRBW, 0><<<dim3(P), dim3(kLmHeadWaves * 64), 0, stream>>>(
        static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, logits, V, logits_bf16, partials, M,
        KT);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  argmax_finalize_kernel<<<dim3(M), dim3(kFinalizeThreads), 0, stream>>>(partials, P, out_idx);
  return hipGetLastError();
}

}  // namespace lsk
