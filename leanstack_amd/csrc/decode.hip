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
#include <mutex>
#include <type_traits>

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

__device__ __forceinline__ float bf16_to_f32(__bf16 v) { return static_cast<float>(v); }

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

// ---------------------------------------------------------------- RMSNorm prologue
//
// y = epilogue(rms_norm(x) . W^T) with rms_norm(x)[m][k] =
// bf16(x[m][k] * nw[k] * r[m]), r[m] = 1 / sqrt(sum_k x[m][k]^2 / K + eps),
// in fp32 with one bf16 rounding -- torch's fused F.rms_norm over the hidden
// dimension (src/leanstack/runtime/qwen_explicit.py:621-628, applied before
// the QKV GEMV at :1255 and before the gate_up GEMV at :941) and the cuTile
// bf16_rmsnorm_kernel (experiments/cutile/qwen_bf16_hot_kernels.py:39-49, its
// torch reference at :52-57), which multiply in the order (x * r) * nw.
// Each wave sums the squares of its own K slice; one LDS exchange gives every
// lane the whole row's sum.

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Sum of the squares of a fragment's 8 values in fp32 (v_dot2c_f32_bf16:
// the bf16 products are exact in fp32).
__device__ __forceinline__ float sum_squares(bf16x8_t v) {
  float s = 0.f;
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), __builtin_shufflevector(v, v, 0, 1), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), __builtin_shufflevector(v, v, 2, 3), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), __builtin_shufflevector(v, v, 4, 5), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), __builtin_shufflevector(v, v, 6, 7), s, false);
  return s;
}

// 1 / sqrt(ss / n + eps) with the mean rounded before eps is added, as
// torch's rms_norm computes it (contraction would fuse the two into an fma).
__device__ __forceinline__ float inv_rms(float ss, int n, float eps) {
#pragma clang fp contract(off)
  return 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
}

// Lanes 0..15 hold this wave's partial sum of squares of rows 0..15; returns
// r[lane % 16] for active rows and 0 for padding columns, summing the waves'
// partials in wave order.  Every wave must call it.
template <int NW>
__device__ __forceinline__ float row_inv_rms(float ss, int wave, int lane, int K, float eps, bool m_active) {
  __shared__ float part[NW][16];
  if (lane < 16) part[wave][lane] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) total += part[w][lane & 15];
  return m_active ? inv_rms(total, K, eps) : 0.f;
}

// bf16((x * nw) * r) of one fragment; `keep` clears padding columns.  The
// product of two bf16 values is exact in fp32, so this is x * nw * r with two
// roundings (fp32, then bf16); the reference's (x * r) * nw differs from it
// by at most one fp32 rounding before the bf16 one.
__device__ __forceinline__ bf16x8_t rms_scale(bf16x8_t xv, bf16x8_t nv, float r, unsigned keep) {
  bf16x8_t o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = static_cast<__bf16>((static_cast<float>(xv[e]) * static_cast<float>(nv[e])) * r);
  u32x4_t bits = __builtin_bit_cast(u32x4_t, o);
  bits &= keep;
  return __builtin_bit_cast(bf16x8_t, bits);
}

// The same from a chunk of x and its 8 norm weights as 4 packed pairs:
// v_dot2c_f32_bf16 of an x pair with a weight pair whose other half is
// masked to zero is the one exact product, so each value costs a mask, a dot
// and a multiply.
__device__ __forceinline__ bf16x8_t rms_scale_pairs(bf16x8_t xv, u32x4_t wv, float r) {
  const u32x4_t xp = __builtin_bit_cast(u32x4_t, xv);
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // Copy the elements out first: this compiler turns __builtin_bit_cast of
    // a vector element with a loop index into a read of element 0.
    const unsigned xe = xp[q], we = wv[q];
    const bf16x2_t xq = __builtin_bit_cast(bf16x2_t, xe);
    const float lo = __builtin_amdgcn_fdot2_f32_bf16(xq, __builtin_bit_cast(bf16x2_t, we & 0x0000ffffu), 0.f, false) * r;
    const float hi = __builtin_amdgcn_fdot2_f32_bf16(xq, __builtin_bit_cast(bf16x2_t, we & 0xffff0000u), 0.f, false) * r;
    o[q] = __builtin_bit_cast(unsigned, bf16x2_t{static_cast<__bf16>(lo), static_cast<__bf16>(hi)});
  }
  return __builtin_bit_cast(bf16x8_t, o);
}

// Dynamic LDS of the single-round RMSNorm prologue: one area per wave.
extern __shared__ __align__(16) unsigned char rms_lds[];

// Bytes of one wave's area in the single-round RMSNorm prologue: the slice's
// norm weights (U*4 chunks of 16 bytes), then the per-chunk sums of squares,
// later overwritten by the M normalised rows of the slice (U * 32 values +
// 8 of padding each).  At the end the wave's partial output tiles
// (RBW x 1 KiB) go to the start of the area for the cross-wave sum.
__host__ __device__ constexpr int rms_wave_bytes(int U, int NC, int M, int RBW) {
  const int stage = U * 4 * 16 + (NC * 64 * 4 > M * (U * 32 + 8) * 2 ? NC * 64 * 4 : M * (U * 32 + 8) * 2);
  return stage > RBW * 1024 ? stage : RBW * 1024;
}

// Single-round accumulate_rows with the RMSNorm prologue (K/32 == NW * U).
// The wave's slice of x -- M rows x U*32 values, M*U*4 chunks of 8 -- is
// spread densely over the lanes, NC chunks per lane, so no lane works for a
// padding column.  Every activation and norm-weight chunk is loaded before
// the weight tiles; the sums of squares, the exchange between waves and the
// scaling run while the weights are in flight.  The normalised rows are
// staged in this wave's LDS area and read back as B fragments.  Sums are
// taken in a fixed order (chunks in K order within a wave, then waves in
// order), so results are bitwise reproducible.  HALF: the half-block form of
// decode_half_kernel (U k-tiles = U/2 pairs; wt is the lane's half-block
// pointer; B column c < M reads row c of tile 2p, M <= c < 2M row c - M of
// tile 2p + 1).
template <int NW, int RBW, int U, int NC, bool HALF = false>
__device__ __forceinline__ void accumulate_rows_rms_dense(f32x4_t (&acc)[RBW], const bf16x8_t* __restrict__ wt,
                                                          const __bf16* __restrict__ x, int ldx,
                                                          const bf16x8_t* __restrict__ nw, int M, int KT, int kb,
                                                          int wave, int lane, float eps) {
  constexpr int kRowChunks = U * 4;     // chunks of 8 values per row of the slice
  static_assert(kRowChunks <= 64, "one lane per norm-weight chunk of the slice");
  constexpr int kRowStride = U * 32 + 8;  // bf16 per staged row: 16 rows start on 16 distinct bank quads
  unsigned char* area = rms_lds + (size_t)wave * rms_wave_bytes(U, NC, M, RBW);
  u32x4_t* nws = reinterpret_cast<u32x4_t*>(area);
  float* ssq = reinterpret_cast<float*>(nws + kRowChunks);
  __bf16* xs = reinterpret_cast<__bf16*>(nws + kRowChunks);
  const int C = M * kRowChunks;
  const int m = lane & 15;
  const int g = lane >> 4;
  const int mr = m < M ? m : M - 1;  // padding columns read row M-1: finite, and never stored

  // Lanes past the last chunk reload it (in bounds); their results are dropped.
  // Lanes 0..U*4-1 also load the slice's norm-weight chunks.
  const bf16x8_t nwc = nw[kb * 4 + min(lane, kRowChunks - 1)];
  bf16x8_t xd[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = min(lane + 64 * i, C - 1);
    const int mc = c / kRowChunks;
    const int j = c - mc * kRowChunks;
    xd[i] = *reinterpret_cast<const bf16x8_t*>(x + (size_t)mc * ldx + (kb * 4 + j) * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  constexpr int kLoads = HALF ? U / 2 : U;  // weight loads per row-block (1 KB each)
  bf16x8_t wv[kLoads][RBW];
#pragma unroll
  for (int u = 0; u < kLoads; ++u) {
#pragma unroll
    for (int r = 0; r < RBW; ++r)
      wv[u][r] = load_weight_tile(wt + ((size_t)r * KT + kb + (HALF ? 2 * u : u)) * 64);
  }
  __builtin_amdgcn_sched_barrier(0);

  // Every lane stores (lanes past the last chunk repeat chunk U*4-1, same
  // value, same slot): a store under `lane < U*4` lets the compiler sink the
  // load into that branch, behind the weight loads, and wait for all of them.
  nws[min(lane, kRowChunks - 1)] = __builtin_bit_cast(u32x4_t, nwc);
  // Straight-line stores (no branch per chunk): slots past C are never read.
#pragma unroll
  for (int i = 0; i < NC; ++i) ssq[lane + 64 * i] = sum_squares(xd[i]);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kRowChunks; ++j) ss += ssq[mr * kRowChunks + j];
  // ssq and xs share the wave's area: these reads of ssq come before the
  // wave's writes of xs in program order, and LDS serves a wave in order.
  const float rr = row_inv_rms<NW>(ss, wave, lane, KT * kTileK, eps, m < M);

#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    const int cc = min(c, C - 1);
    const int mc = cc / kRowChunks;
    const int j = cc - mc * kRowChunks;
    const float rc = __shfl(rr, mc);  // lane mc < 16 holds r of row mc
    const bf16x8_t o = rms_scale_pairs(xd[i], nws[j], rc);
    // Lanes past the last chunk store the last chunk's own value again.
    *reinterpret_cast<bf16x8_t*>(xs + mc * kRowStride + j * 8) = o;
  }
  if constexpr (HALF) {
    // Column m: row m of the even tile, row m - M of the odd one; columns
    // past 2M read row M-1 (finite, never stored).
    const int hi = m >= M && m < 2 * M ? 1 : 0;
    const int row = m < M ? m : (hi ? m - M : M - 1);
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const bf16x8_t xn = *reinterpret_cast<const bf16x8_t*>(xs + row * kRowStride + (2 * u + hi) * 32 + g * 8);
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xn, acc[r]);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bf16x8_t xn = *reinterpret_cast<const bf16x8_t*>(xs + mr * kRowStride + u * 32 + g * 8);
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xn, acc[r]);
    }
  }
}

// Bytes of one wave's area when its slice of x is staged: the M rows of the
// slice (row stride U*32+8 bf16), and at least the RBW partial tiles of the
// cross-wave sum that reuse the area.
__host__ __device__ constexpr int staged_wave_bytes(int U, int M, int RBW) {
  return M * (U * 32 + 8) * 2 > RBW * 1024 ? M * (U * 32 + 8) * 2 : RBW * 1024;
}

// NORM value of the kernels' staged-activation form with NC chunks per lane
// (NORM = 0: fragments loaded per tile; > 0 and -1: the RMSNorm prologues).
constexpr int staged_x(int nc) { return -1 - nc; }
// The same with the wave's x slice staged in two phases (NC chunks per lane
// per phase): decode_linear_kernel only.
constexpr int staged_x2(int nc) { return -101 - nc; }

// Single-round accumulate_rows with the wave's slice of x -- M rows x U*32
// values, M*U*4 chunks of 8 -- loaded densely (NC chunks per lane, one
// request per chunk) and staged in the wave's LDS area, then read back as B
// fragments.  Loading the fragments per tile instead makes every lane of
// every wave request 16 bytes per k-tile, padding columns included: at M = 1
// as many vector-memory requests as the weight tiles themselves.  HALF: the
// half-block fragment order (see accumulate_rows_rms_dense).  No barrier:
// each wave reads only its own area.
template <int NW, int RBW, int U, int NC, bool HALF, int PH = 1>
__device__ __forceinline__ void accumulate_rows_staged(f32x4_t (&acc)[RBW], const bf16x8_t* __restrict__ wt,
                                                       const __bf16* __restrict__ x, int ldx, int M, int KT, int kb,
                                                       int wave, int lane) {
  static_assert(PH == 1 || (PH == 2 && !HALF), "two-phase staging is for the 16-row form");
  constexpr int kRowStride = U * 32 + 8;
  __bf16* xs = reinterpret_cast<__bf16*>(rms_lds + (size_t)wave * staged_wave_bytes(U, M, RBW));
  const int m = lane & 15;
  const int g = lane >> 4;
  // Phase p stages k-tiles [kt0(p), kt0(p + 1)) of the wave's slice: M rows
  // of (kt1 - kt0) * 4 chunks of 8 values, NC chunks per lane.
  auto kt0 = [](int p) { return p * U / PH; };
  bf16x8_t xd[NC];
  auto load_phase = [&](int p) {
    const int pc = (kt0(p + 1) - kt0(p)) * 4;
    const int C = M * pc;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(lane + 64 * i, C - 1);  // lanes past the last chunk reload it
      const int mc = c / pc;
      const int j = kt0(p) * 4 + c - mc * pc;
      xd[i] = *reinterpret_cast<const bf16x8_t*>(x + (size_t)mc * ldx + (kb * 4 + j) * 8);
    }
  };
  auto store_phase = [&](int p) {
    const int pc = (kt0(p + 1) - kt0(p)) * 4;
    const int C = M * pc;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = min(lane + 64 * i, C - 1);
      const int mc = c / pc;
      const int j = kt0(p) * 4 + c - mc * pc;
      *reinterpret_cast<bf16x8_t*>(xs + mc * kRowStride + j * 8) = xd[i];
    }
  };
  load_phase(0);
  __builtin_amdgcn_sched_barrier(0);
  constexpr int kLoads = HALF ? U / 2 : U;
  bf16x8_t wv[kLoads][RBW];
#pragma unroll
  for (int u = 0; u < kLoads; ++u) {
#pragma unroll
    for (int r = 0; r < RBW; ++r)
      wv[u][r] = load_weight_tile(wt + ((size_t)r * KT + kb + (HALF ? 2 * u : u)) * 64);
  }
  __builtin_amdgcn_sched_barrier(0);
  store_phase(0);
  if constexpr (HALF) {
    const int hi = m >= M && m < 2 * M ? 1 : 0;
    const int row = m < M ? m : (hi ? m - M : M - 1);
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const bf16x8_t xn = *reinterpret_cast<const bf16x8_t*>(xs + row * kRowStride + (2 * u + hi) * 32 + g * 8);
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xn, acc[r]);
    }
  } else {
    const int mr = m < M ? m : M - 1;  // padding columns: finite, never stored
    // The second phase's chunks load while the first phase multiplies (they
    // queue behind the weight loads, which the first multiplies wait for).
    if constexpr (PH == 2) load_phase(1);
#pragma unroll
    for (int p = 0; p < PH; ++p) {
      if (p == 1) store_phase(1);
#pragma unroll
      for (int u = kt0(p); u < kt0(p + 1); ++u) {
        const bf16x8_t xn = *reinterpret_cast<const bf16x8_t*>(xs + mr * kRowStride + u * 32 + g * 8);
#pragma unroll
        for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xn, acc[r]);
      }
    }
  }
}

// Round-based accumulate_rows with the RMSNorm prologue (any K): a first pass
// over the wave's activation fragments (cache hits) gives r, then the rounds
// run as in accumulate_rows with each fragment scaled before its multiply.
// nrow: norm weight as 16-byte units, + g (the index pattern of xrow).
template <int NW, int RBW>
__device__ __forceinline__ void accumulate_rows_rms(f32x4_t (&acc)[RBW], const bf16x8_t* __restrict__ wt,
                                                    const bf16x8_t* __restrict__ xrow,
                                                    const bf16x8_t* __restrict__ nrow, bool m_active, int KT,
                                                    int kb, int ke, int wave, int lane, float eps) {
  const unsigned keep = m_active ? 0xffffffffu : 0u;
  float ss = 0.f;
  for (int kt = kb; kt < ke; ++kt) ss += sum_squares(xrow[kt * 4]);
  // lanes m, m+16, m+32, m+48 hold the four K groups of row m
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  const float rr = row_inv_rms<NW>(ss, wave, lane, KT * kTileK, eps, m_active);
  constexpr int R = 8 / RBW;
  int kt = kb;
  for (; kt + R <= ke; kt += R) {
    bf16x8_t xv[R], nv[R];
    bf16x8_t wv[R][RBW];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      xv[u] = xrow[(kt + u) * 4];
      nv[u] = nrow[(kt + u) * 4];
#pragma unroll
      for (int r = 0; r < RBW; ++r) wv[u][r] = load_weight_tile(wt + ((size_t)r * KT + kt + u) * 64);
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const bf16x8_t xn = rms_scale(xv[u], nv[u], rr, keep);
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xn, acc[r]);
    }
  }
  for (; kt < ke; ++kt) {
    const bf16x8_t xn = rms_scale(xrow[kt * 4], nrow[kt * 4], rr, keep);
#pragma unroll
    for (int r = 0; r < RBW; ++r) acc[r] = mfma16(load_weight_tile(wt + ((size_t)r * KT + kt) * 64), xn, acc[r]);
  }
}

// The same with wave w's tiles at base + w * stride (w >= 1): its own area
// of the RMSNorm prologue, which it has finished reading.
template <int NW, int RBW>
__device__ __forceinline__ bool reduce_waves_at(f32x4_t (&acc)[RBW], int wave, int lane, unsigned char* base,
                                                int stride) {
  if (wave > 0) {
    f32x4_t* t = reinterpret_cast<f32x4_t*>(base + (size_t)wave * stride);
#pragma unroll
    for (int r = 0; r < RBW; ++r) t[r * 64 + lane] = acc[r];
  }
  __syncthreads();
  if (wave != 0) return false;
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    const f32x4_t* t = reinterpret_cast<const f32x4_t*>(base + (size_t)w * stride);
#pragma unroll
    for (int r = 0; r < RBW; ++r) acc[r] += t[r * 64 + lane];
  }
  return true;
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

// y = epilogue(x . W^T) for M <= 16, or epilogue(rms_norm(x) . W^T) with
// NORM != 0: NORM > 0 is the single-round prologue with NORM chunks per lane
// (U > 0, dynamic LDS of NW * rms_wave_bytes(U, NORM, M, RBW) bytes), NORM < 0
// the round-based one (U == 0).  Grid: (NB / RBW) workgroups of NW waves;
// U > 0 requires K/32 == NW * U (single-round loads).
template <int NW, int RBW, int EPI, int U, int NORM>
__global__ __launch_bounds__(NW * 64) void decode_linear_kernel(
    const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x, int ldx, __bf16* __restrict__ y,
    int ldy, const __bf16* __restrict__ residual, int ldr, int M, int KT, const __bf16* __restrict__ norm_w,
    float eps) {
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

  // Residual values of the outputs wave 0 will write, read before the
  // weight stream so that their latency is not paid after the cross-wave
  // sum (rows past M read row 0: in bounds, never stored).
  float res[RBW][4];
  if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd)) {
    if (wave == 0) {
#pragma unroll
      for (int r = 0; r < RBW; ++r) {
        const __bf16* rp = residual + (size_t)(m_active ? m : 0) * ldr + (rb0 + r) * 16 + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) res[r][i] = bf16_to_f32(rp[i]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  const bf16x8_t* xrow = reinterpret_cast<const bf16x8_t*>(x + (size_t)(m_active ? m : 0) * ldx) + g;
  const bf16x8_t* wt = w + (size_t)rb0 * KT * 64 + lane;
  static_assert(NORM <= 0 || U > 0, "the dense RMSNorm prologue is single-round");
  static_assert(NORM != -1 || U == 0, "the per-lane RMSNorm prologue is round-based");
  static_assert(NORM >= -1 || U > 0, "staged activations are single-round");
  if constexpr (NORM > 0) {
    accumulate_rows_rms_dense<NW, RBW, U, NORM>(acc, wt, x, ldx, reinterpret_cast<const bf16x8_t*>(norm_w), M, KT,
                                                kb, wave, lane, eps);
  } else if constexpr (NORM == -1) {
    const bf16x8_t* nrow = reinterpret_cast<const bf16x8_t*>(norm_w) + g;
    accumulate_rows_rms<NW, RBW>(acc, wt, xrow, nrow, m_active, KT, kb, ke, wave, lane, eps);
  } else if constexpr (NORM < -100) {
    (void)norm_w;
    (void)eps;
    accumulate_rows_staged<NW, RBW, U, -101 - NORM, false, 2>(acc, wt, x, ldx, M, KT, kb, wave, lane);
  } else if constexpr (NORM < -1) {
    (void)norm_w;
    (void)eps;
    accumulate_rows_staged<NW, RBW, U, -1 - NORM, false>(acc, wt, x, ldx, M, KT, kb, wave, lane);
  } else {
    (void)norm_w;
    (void)eps;
    accumulate_rows<RBW, U>(acc, wt, xrow, m_active, KT, kb, ke);
  }

  if constexpr (NORM > 0) {
    if (!reduce_waves_at<NW, RBW>(acc, wave, lane, rms_lds, rms_wave_bytes(U, NORM, M, RBW))) return;
  } else if constexpr (NORM < -1) {
    if (!reduce_waves_at<NW, RBW>(acc, wave, lane, rms_lds, staged_wave_bytes(U, M, RBW))) return;
  } else {
    if (!reduce_waves<NW, RBW>(acc, wave, lane)) return;
  }
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
        if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd)) v = res[r][i] + v;
        o[i] = bf16_bits(v);
      }
      *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + n) =
          u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
    }
  }
}

// The order torch.argmax reduces in: NaN above every number (the first NaN
// wins), then the larger value, then the lower index among equal values.  An
// all -inf row therefore yields its first index, never the INT_MAX of an
// empty candidate, so the token id is always a valid vocab row.
__device__ __forceinline__ bool argmax_beats(float s, int i, float best, int best_idx) {
  const bool s_nan = s != s;
  const bool b_nan = best != best;
  if (s_nan != b_nan) return s_nan;
  if (!s_nan && s != best) return s > best;
  return i < best_idx;
}

__device__ __forceinline__ void argmax_take(float& best, int& best_idx, float s, int i) {
  if (argmax_beats(s, i, best, best_idx)) {
    best = s;
    best_idx = i;
  }
}

typedef __attribute__((address_space(1))) unsigned long long global_u64_t;

// The argmax partials live in the workspace as 64-bit words: the score's bits
// in the low half and index + 1 in the high half, so a word that is zero has
// not been written by this call yet (between calls every word is zero).
// Stores and loads are device-coherent: partials cross XCDs.
__device__ __forceinline__ void store_partial(ArgmaxPartial* p, float score, int index) {
  const unsigned long long v =
      (unsigned long long)__builtin_bit_cast(unsigned, score) | ((unsigned long long)(unsigned)(index + 1) << 32);
  __hip_atomic_store((global_u64_t*)(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long load_partial(const ArgmaxPartial* p) {
  return __hip_atomic_load((const global_u64_t*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr unsigned kHeadSpinLimit = 1u << 20;  // polls of one partial before the second stage gives up
constexpr int kRoundLoads = 10;  // partial loads in flight per thread of the second stage

// Second stage of the greedy head, as the host-side torch.argmax over tile
// maxima in src/leanstack/runtime/cutile_logits.py:67-69: the NT threads of
// one workgroup reduce the P partials of one activation row into *out, then
// zero them for the next call.  Every load of a round is issued before the
// first compare; a partial still zero (its workgroup has not stored it) is
// polled again.  argmax_take is a total order on (score, index), so the
// result does not depend on the order partials are combined in.  A partial
// that stays zero for kHeadSpinLimit polls makes the row's result -1 and
// counts one give-up in *status (neither happens while every workgroup of
// the grid runs to its end, which nothing in the grid waits on).
template <int NT>
__device__ __forceinline__ void reduce_row_partials(ArgmaxPartial* __restrict__ row, int P,
                                                    long long* __restrict__ out, unsigned* __restrict__ status) {
  constexpr int kW = NT / 64;
  __shared__ float s_best[kW];
  __shared__ int s_idx[kW];
  __shared__ int s_gave_up[kW];
  const int t = (int)threadIdx.x;
  float best = -__builtin_huge_valf();
  int best_idx = INT_MAX;
  bool gave_up = false;
  for (int base = 0; base < P; base += NT * kRoundLoads) {
    unsigned long long v[kRoundLoads];
#pragma unroll
    for (int j = 0; j < kRoundLoads; ++j) {
      const int p = base + j * NT + t;
      v[j] = p < P ? load_partial(row + p) : 0ull;
    }
#pragma unroll
    for (int j = 0; j < kRoundLoads; ++j) {
      const int p = base + j * NT + t;
      if (p >= P) continue;
      for (unsigned spins = 0; (v[j] >> 32) == 0;) {
        if (++spins > kHeadSpinLimit) {
          gave_up = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        v[j] = load_partial(row + p);
      }
      __hip_atomic_store((global_u64_t*)(row + p), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((v[j] >> 32) != 0)
        argmax_take(best, best_idx, __builtin_bit_cast(float, (unsigned)v[j]), (int)(v[j] >> 32) - 1);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float os = __shfl_xor(best, off);
    const int oi = __shfl_xor(best_idx, off);
    argmax_take(best, best_idx, os, oi);
  }
  const bool wave_gave_up = __any(gave_up);
  if ((t & 63) == 0) {
    s_best[t >> 6] = best;
    s_idx[t >> 6] = best_idx;
    s_gave_up[t >> 6] = wave_gave_up;
  }
  __syncthreads();
  if (t == 0) {
    bool any_gave_up = false;
    for (int w = 0; w < kW; ++w) {
      argmax_take(best, best_idx, s_best[w], s_idx[w]);
      any_gave_up |= s_gave_up[w] != 0;
    }
    *out = any_gave_up ? -1 : best_idx;
    if (any_gave_up) __hip_atomic_fetch_add(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// lm_head scores for RB row-blocks (vocab rows) from row-block rb0, and their
// best (score, index) per activation row stored as partial[m * P + slot].
// NC > 0: the activations staged through LDS (NC chunks per lane), or with
// NORM their RMSNorm (norm_w, eps) applied on the way (the dense prologue).
template <int NW, int RB, int U, int NC, bool NORM>
__device__ __forceinline__ void lm_head_score(const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x, int ldx,
                                              float* __restrict__ logits, int V, int logits_bf16,
                                              ArgmaxPartial* __restrict__ partial, int P, int M, int KT,
                                              const __bf16* __restrict__ norm_w, float eps, int rb0, int slot) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = lane & 15;
  const int g = lane >> 4;
  const bool m_active = m < M;
  const int kb = (KT * wave) / NW;
  const int ke = (KT * (wave + 1)) / NW;

  f32x4_t acc[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bf16x8_t* xrow = reinterpret_cast<const bf16x8_t*>(x + (size_t)(m_active ? m : 0) * ldx) + g;
  const bf16x8_t* wt = w + (size_t)rb0 * KT * 64 + lane;
  bool leader;  // wave 0, which holds the sums after reduce_waves
  if constexpr (NORM) {
    (void)xrow;
    (void)ke;
    accumulate_rows_rms_dense<NW, RB, U, NC>(acc, wt, x, ldx, reinterpret_cast<const bf16x8_t*>(norm_w), M, KT,
                                              kb, wave, lane, eps);
    leader = reduce_waves_at<NW, RB>(acc, wave, lane, rms_lds, rms_wave_bytes(U, NC, M, RB));
  } else if constexpr (NC > 0) {  // activations staged through LDS, NC chunks per lane
    (void)xrow;
    (void)ke;
    (void)norm_w;
    (void)eps;
    accumulate_rows_staged<NW, RB, U, NC, false>(acc, wt, x, ldx, M, KT, kb, wave, lane);
    leader = reduce_waves_at<NW, RB>(acc, wave, lane, rms_lds, staged_wave_bytes(U, M, RB));
  } else {
    (void)norm_w;
    (void)eps;
    accumulate_rows<RB, U>(acc, wt, xrow, m_active, KT, kb, ke);
    leader = reduce_waves<NW, RB>(acc, wave, lane);
  }

  if (leader) {
    // Scan this lane's rows in increasing index order with the torch.argmax
    // order (argmax_beats): every row, -inf and NaN included, gets a real index.
    float best = -__builtin_huge_valf();
    int best_idx = INT_MAX;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int n0 = (rb0 + r) * 16 + 4 * g;
      f32x4_t s = acc[r];
      if (logits_bf16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = bf16_round(s[i]);
      }
      if (logits != nullptr && m_active) *reinterpret_cast<f32x4_t*>(logits + (size_t)m * V + n0) = s;
#pragma unroll
      for (int i = 0; i < 4; ++i) argmax_take(best, best_idx, s[i], n0 + i);
    }
    // Lanes m, m+16, m+32, m+48 hold the same column: combine them.
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const float os = __shfl_xor(best, off);
      const int oi = __shfl_xor(best_idx, off);
      argmax_take(best, best_idx, os, oi);
    }
    if (g == 0 && m_active) store_partial(partial + (size_t)m * P + slot, best, best_idx);
  }
}

// lm_head scores + the argmax, in one launch.  Grid: P scoring workgroups,
// then M reducing ones (lm_head_partials).  The first P2 scoring workgroups
// take RBW row-blocks each and the last P - P2 one each, so that the grid's
// last workgroups are short and finish close together (the CUs otherwise
// idle through the end of the last long ones); NB = RBW * P2 + (P - P2).
// Scoring workgroup b stores partial[m * P + b] = its best (score, index)
// for row m; reducing workgroup P + m -- dispatched after every scoring one,
// so it waits only for workgroups that are running or done -- reduces row m
// into out_idx[m] while the last scoring workgroups finish
// (reduce_row_partials).  The workspace must be zero when a call starts, and
// every call leaves it zero.
template <int NW, int RBW, int U, int NC = 0, bool NORM = false>
__global__ __launch_bounds__(NW * 64) void lm_head_kernel(
    const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x, int ldx, float* __restrict__ logits,
    int V, int logits_bf16, ArgmaxPartial* __restrict__ partial, unsigned* __restrict__ status,
    long long* __restrict__ out_idx, int M, int KT, const __bf16* __restrict__ norm_w, float eps) {
  static_assert(!NORM || NC > 0, "the RMSNorm prologue is the dense single-round one");
  const int P = (int)gridDim.x - M;
  const int b = (int)blockIdx.x;
  if (b >= P) {
    const int row = b - P;
    reduce_row_partials<NW * 64>(partial + (size_t)row * P, P, out_idx + row, status);
    return;
  }
  if constexpr (RBW == 1) {
    lm_head_score<NW, 1, U, NC, NORM>(w, x, ldx, logits, V, logits_bf16, partial, P, M, KT, norm_w, eps, b, b);
  } else {
    const int P2 = (V / kTileRows - P) / (RBW - 1);
    if (b < P2)
      lm_head_score<NW, RBW, U, NC, NORM>(w, x, ldx, logits, V, logits_bf16, partial, P, M, KT, norm_w, eps,
                                          b * RBW, b);
    else
      lm_head_score<NW, 1, U, NC, NORM>(w, x, ldx, logits, V, logits_bf16, partial, P, M, KT, norm_w, eps,
                                        P2 * RBW + (b - P2), b);
  }
}

constexpr int kLmHeadWaves = 8;
constexpr int kLmHeadRBW = 2;

// Launch arguments of one decode / verify projection.
struct DecodeArgs {
  const void* w;
  int NB, KT;
  const void* x;
  int M, ldx;
  void* y;
  int ldy;
  const void* residual;
  int ldr;
  const void* norm_w;  // RMSNorm weight [K], or null
  float eps;
};

// Dynamic LDS a launch may use without raising the kernel's limit first.
constexpr size_t kDefaultDynamicLds = 64 * 1024;

template <int NW, int RBW, int EPI, int U, int NORM>
hipError_t launch_decode_cfg(const DecodeArgs& a, hipStream_t stream) {
  auto* kernel = decode_linear_kernel<NW, RBW, EPI, U, NORM>;
  size_t lds = NORM < -1 ? (size_t)NW * staged_wave_bytes(U, a.M, RBW) : 0;
  if constexpr (NORM < -1) {
    if (lds > kDefaultDynamicLds) {
      // Raised once per kernel, to what M = 8 (the largest staged M) needs.
      static std::once_flag once;
      static hipError_t raised = hipSuccess;
      std::call_once(once, [&] {
        raised = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     NW * staged_wave_bytes(U, 8, RBW));
      });
      if (raised != hipSuccess) return raised;
    }
  }
  if constexpr (NORM > 0) {
    lds = (size_t)NW * rms_wave_bytes(U, NORM, a.M, RBW);
    if (lds > kDefaultDynamicLds) {
      // Raised once per kernel, to what M = 16 needs.
      static std::once_flag once;
      static hipError_t raised = hipSuccess;
      std::call_once(once, [&] {
        raised = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     NW * rms_wave_bytes(U, NORM, kDecodeMaxM, RBW));
      });
      if (raised != hipSuccess) return raised;
    }
  }
  launch_kernel(kernel, dim3(a.NB / RBW), dim3(NW * 64), lds, stream,
      static_cast<const bf16x8_t*>(a.w), static_cast<const __bf16*>(a.x), a.ldx, static_cast<__bf16*>(a.y), a.ldy,
      static_cast<const __bf16*>(a.residual), a.ldr, a.M, a.KT, static_cast<const __bf16*>(a.norm_w), a.eps);
  return hipGetLastError();
}

// Half-block form for M <= 8: workgroup b covers rows 8h .. 8h+7 (h = b & 1)
// of row-block(s) (b >> 1) * RBW .., so a projection has twice as many,
// half-sized workgroups.  One wave load still moves 1 KB of whole 128-byte
// lines: lanes with c < 8 read the 8 rows of k-tile 2p (their chunks of a
// packed tile are lines 0, 2, 4, 6 or 1, 3, 5, 7), lanes with c >= 8 the
// same rows of k-tile 2p + 1.  The activation fragments of tile 2p go to B
// columns 0..M-1, those of tile 2p + 1 to columns M..2M-1, so output row
// 8h + i (i < 8) of x row m is D[i][m] + D[8 + i][M + m] (even tiles plus
// odd tiles, added once after the wave reduction).  Grid: 2 * NB / RBW
// workgroups of NW waves; K/32 == 2 * NW * U (single-round loads).
// With 16-row workgroups the QKV projection (384 row-blocks) leaves half of
// the 256 CUs with one workgroup and half with two, and gate_up (608 pairs)
// runs a third round on 96 CUs; halves make 3 per CU and 4.75 per CU.
template <int NW, int RBW, int EPI, int U, int NORM>
__global__ __launch_bounds__(NW * 64) void decode_half_kernel(
    const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x, int ldx, __bf16* __restrict__ y,
    int ldy, const __bf16* __restrict__ residual, int ldr, int M, int KT, const __bf16* __restrict__ norm_w,
    float eps) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int h = blockIdx.x & 1;
  const int rb0 = (blockIdx.x >> 1) * RBW;
  const bf16x8_t* wt = w + (size_t)rb0 * KT * 64 + (c >> 3) * 64 + g * 16 + 8 * h + (c & 7);
  const bool b_lo = c < M;
  const bool b_hi = c >= M && c < 2 * M;
  const unsigned keep = (b_lo || b_hi) ? 0xffffffffu : 0u;
  const int xr = b_lo ? c : (b_hi ? c - M : 0);
  const bf16x8_t* xrow = reinterpret_cast<const bf16x8_t*>(x + (size_t)xr * ldx) + (b_hi ? 4 : 0) + g;
  f32x4_t acc[RBW];
#pragma unroll
  for (int r = 0; r < RBW; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int pb = wave * U;
  if constexpr (NORM > 0) {
    (void)xrow;
    (void)keep;
    accumulate_rows_rms_dense<NW, RBW, 2 * U, NORM, true>(acc, wt, x, ldx, reinterpret_cast<const bf16x8_t*>(norm_w),
                                                          M, KT, 2 * pb, wave, lane, eps);
    if (!reduce_waves_at<NW, RBW>(acc, wave, lane, rms_lds, rms_wave_bytes(2 * U, NORM, M, RBW))) return;
  } else if constexpr (NORM < -1) {
    (void)xrow;
    (void)keep;
    (void)norm_w;
    (void)eps;
    accumulate_rows_staged<NW, RBW, 2 * U, -1 - NORM, true>(acc, wt, x, ldx, M, KT, 2 * pb, wave, lane);
    if (!reduce_waves_at<NW, RBW>(acc, wave, lane, rms_lds, staged_wave_bytes(2 * U, M, RBW))) return;
  } else {
    (void)norm_w;
    (void)eps;
    bf16x8_t wv[U][RBW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int r = 0; r < RBW; ++r) wv[u][r] = load_weight_tile(wt + ((size_t)r * KT + 2 * (pb + u)) * 64);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bf16x8_t xv = load_x_frag(xrow + (pb + u) * 8, keep);
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(wv[u][r], xv, acc[r]);
    }
    if (!reduce_waves<NW, RBW>(acc, wave, lane)) return;
  }
  const int partner = lane + 32 + M;  // only read where g < 2 and c < M (partner < 64)
#pragma unroll
  for (int r = 0; r < RBW; ++r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[r][i] += __shfl(acc[r][i], partner & 63);
  }
  if (g >= 2 || c >= M) return;
  const int m = c;
  if constexpr (EPI == static_cast<int>(Epilogue::kSiluMul)) {
    const int j = (blockIdx.x >> 1) * 16 + 8 * h + 4 * g;
    unsigned short o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = bf16_bits(silu_mul_bf16(acc[0][i], acc[1][i]));
    *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + j) =
        u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
  } else {
#pragma unroll
    for (int r = 0; r < RBW; ++r) {
      const int n = (rb0 + r) * 16 + 8 * h + 4 * g;
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

template <int NW, int RBW, int EPI, int U, int NORM = 0>
hipError_t launch_half_cfg(const DecodeArgs& a, hipStream_t stream) {
  const size_t lds = NORM > 0    ? (size_t)NW * rms_wave_bytes(2 * U, NORM, a.M, RBW)
                     : NORM < -1 ? (size_t)NW * staged_wave_bytes(2 * U, a.M, RBW)
                                 : 0;
  launch_kernel(decode_half_kernel<NW, RBW, EPI, U, NORM>, dim3(a.NB / RBW * 2), dim3(NW * 64), lds, stream,
      static_cast<const bf16x8_t*>(a.w), static_cast<const __bf16*>(a.x), a.ldx, static_cast<__bf16*>(a.y), a.ldy,
      static_cast<const __bf16*>(a.residual), a.ldr, a.M, a.KT, static_cast<const __bf16*>(a.norm_w), a.eps);
  return hipGetLastError();
}

// The staged-activation form with NC (1..8) chunks per lane; HALF selects
// decode_half_kernel (U = pairs per wave), else decode_linear_kernel.
template <int NW, int RBW, int EPI, int U, bool HALF>
hipError_t launch_staged(const DecodeArgs& a, int nc, hipStream_t stream) {
  auto go = [&](auto tag) -> hipError_t {
    constexpr int kNorm = staged_x(decltype(tag)::value);
    if constexpr (HALF) return launch_half_cfg<NW, RBW, EPI, U, kNorm>(a, stream);
    else return launch_decode_cfg<NW, RBW, EPI, U, kNorm>(a, stream);
  };
  switch (nc) {
    case 1:
      return go(std::integral_constant<int, 1>{});
    case 2:
      return go(std::integral_constant<int, 2>{});
    case 3:
      return go(std::integral_constant<int, 3>{});
    case 4:
      return go(std::integral_constant<int, 4>{});
    case 5:
      return go(std::integral_constant<int, 5>{});
    case 6:
      return go(std::integral_constant<int, 6>{});
    case 7:
      return go(std::integral_constant<int, 7>{});
    case 8:
      return go(std::integral_constant<int, 8>{});
    default:
      return hipErrorInvalidValue;
  }
}

// Shape dispatch: the Qwen3-4B K values get single-round instantiations
// (K/32 = 80 -> 16 waves x 5 for QKV and the gate/up pairs, 128 -> 8 x 16,
// 304 -> 16 x 19, each measured faster than the alternatives on MI355X); any
// other K runs the round-based variant.
template <int RBW, int EPI>
hipError_t launch_decode_shape(const DecodeArgs& a, hipStream_t stream) {
  // K/32 = 80 at M <= 8 (QKV and gate_up, 36-layer step at M = 1):
  // half-blocks, QKV 8 waves x 5 pairs, gate_up 4 waves x 10 pairs; measured
  // 55 us (3.6 %) faster per step than 16-row workgroups.  o_proj and down
  // (160 row-blocks) measured slower as halves: 320 workgroups leave 64 CUs
  // with two.
  // Activations staged through LDS (staged_x(NC), NC = chunks per lane of
  // the wave's M * 4 * k-tiles chunks) wherever the registers allow: QKV and
  // o_proj for every M <= 8, gate_up (4 waves x 10 pairs up to M = 2, then
  // 8 waves x 5), down in one phase up to M = 5 and in two from M = 6 (its
  // 16 waves hold up to 154 KB of LDS at M = 8).
  if (a.KT == 80 && a.M <= 8) {
    if constexpr (RBW == 1) return launch_staged<8, RBW, EPI, 5, true>(a, (40 * a.M + 63) / 64, stream);
    if constexpr (RBW == 2) {
      if (a.M <= 2) return launch_staged<4, RBW, EPI, 10, true>(a, (80 * a.M + 63) / 64, stream);
      return launch_staged<8, RBW, EPI, 5, true>(a, (40 * a.M + 63) / 64, stream);
    }
  }
  if constexpr (RBW == 1) {
    if (a.KT == 128 && a.M <= 8) return launch_staged<8, RBW, EPI, 16, false>(a, a.M, stream);
    if (a.KT == 304 && a.M <= 5) return launch_staged<16, RBW, EPI, 19, false>(a, (76 * a.M + 63) / 64, stream);
    // M = 6..8: in two phases (10 + 9 k-tiles, 4 or 5 chunks per lane each),
    // so the chunk registers fit beside the 19 weight tiles (8-10 chunks in
    // one phase spill): 13.7-14.3 -> 11.5-11.9 us per launch; at M = 5 the
    // single phase (6 chunks) is 0.3 us faster.
    if (a.KT == 304 && a.M <= 6) return launch_decode_cfg<16, RBW, EPI, 19, staged_x2(4)>(a, stream);
    if (a.KT == 304 && a.M <= 8) return launch_decode_cfg<16, RBW, EPI, 19, staged_x2(5)>(a, stream);
  }
  if (a.KT == 80 && a.M <= 8) {
    if constexpr (RBW == 1) return launch_half_cfg<8, RBW, EPI, 5>(a, stream);
    if constexpr (RBW == 2) return launch_half_cfg<4, RBW, EPI, 10>(a, stream);
  }
  switch (a.KT) {
    case 80:
      // (M > 8) 16 waves x 5 k-tiles, for the single row-block (QKV) and the
      // gate/up pair alike: measured 4.5 % / 3.2 % faster than 8 waves x 10 (whose
      // gate/up form needs 96 VGPRs and leaves 96 of 608 workgroups for a
      // second wave) and than the round-based loop.
      return launch_decode_cfg<16, RBW, EPI, 5, 0>(a, stream);
    case 128:
      if constexpr (RBW == 1) return launch_decode_cfg<8, RBW, EPI, 16, 0>(a, stream);
      break;
    case 304:
      if constexpr (RBW == 1) return launch_decode_cfg<16, RBW, EPI, 19, 0>(a, stream);
      break;
    default:
      break;
  }
  if (a.KT >= 256) return launch_decode_cfg<16, RBW, EPI, 0, 0>(a, stream);
  return launch_decode_cfg<8, RBW, EPI, 0, 0>(a, stream);
}

// The same with the RMSNorm prologue.  K/32 = 80 (the Qwen3-4B hidden size
// the norms act on) runs single-round with the dense prologue, its chunks
// per lane (M * 20 chunks over 64 lanes) picked from M; any other K runs
// the round-based prologue.
template <int RBW, int EPI>
hipError_t launch_rms_shape(const DecodeArgs& a, hipStream_t stream) {
  // Half-blocks for M <= 8, 8 waves x 5 pairs (10 k-tiles, 40 norm-weight
  // chunks per wave): chunks per lane = ceil(40 M / 64).
  if (a.KT == 80 && a.M <= 8) {
    if (a.M == 1) return launch_half_cfg<8, RBW, EPI, 5, 1>(a, stream);
    if (a.M <= 3) return launch_half_cfg<8, RBW, EPI, 5, 2>(a, stream);
    if (a.M == 4) return launch_half_cfg<8, RBW, EPI, 5, 3>(a, stream);
    if (a.M <= 6) return launch_half_cfg<8, RBW, EPI, 5, 4>(a, stream);
    return launch_half_cfg<8, RBW, EPI, 5, 5>(a, stream);
  }
  if (a.KT == 80) {
    if (a.M <= 3) return launch_decode_cfg<16, RBW, EPI, 5, 1>(a, stream);
    if (a.M <= 9) return launch_decode_cfg<16, RBW, EPI, 5, 3>(a, stream);
    return launch_decode_cfg<16, RBW, EPI, 5, 5>(a, stream);
  }
  if (a.KT >= 256) return launch_decode_cfg<16, RBW, EPI, 0, -1>(a, stream);
  return launch_decode_cfg<8, RBW, EPI, 0, -1>(a, stream);
}

template <bool NORM>
hipError_t launch_decode_epi(const DecodeArgs& a, Epilogue epi, hipStream_t stream) {
  switch (epi) {
    case Epilogue::kSiluMul:
      return NORM ? launch_rms_shape<2, 1>(a, stream) : launch_decode_shape<2, 1>(a, stream);
    case Epilogue::kResidualAdd:
      return NORM ? launch_rms_shape<1, 2>(a, stream) : launch_decode_shape<1, 2>(a, stream);
    case Epilogue::kNone:
    default:
      return NORM ? launch_rms_shape<1, 0>(a, stream) : launch_decode_shape<1, 0>(a, stream);
  }
}

}  // namespace

hipError_t launch_decode_linear(const void* w, int N, int K, const void* x, int M, int ldx, void* y,
                                int ldy, Epilogue epi, const void* residual, int ldr, hipStream_t stream) {
  const DecodeArgs a{w, N / kTileRows, K / kTileK, x, M, ldx, y, ldy, residual, ldr, nullptr, 0.f};
  return launch_decode_epi<false>(a, epi, stream);
}

hipError_t launch_decode_rmsnorm_linear(const void* w, int N, int K, const void* x, int M, int ldx,
                                        const void* norm_w, float eps, void* y, int ldy, Epilogue epi,
                                        const void* residual, int ldr, hipStream_t stream) {
  const DecodeArgs a{w, N / kTileRows, K / kTileK, x, M, ldx, y, ldy, residual, ldr, norm_w, eps};
  return launch_decode_epi<true>(a, epi, stream);
}

// Single-row-block workgroups at the end of the lm_head grid: 2 per CU of a
// 256-CU MI355X (measured at V = 151936, M = 1: 115.1 -> 113.9 us; a tail of
// 384, 768 or 1024 was no better).
constexpr int kLmHeadTail = 512;

int lm_head_partials(int V) {
  const int NB = V / kTileRows;
  if (kLmHeadRBW == 1 || NB <= kLmHeadTail) return NB;
  const int tail = kLmHeadTail + (NB - kLmHeadTail) % kLmHeadRBW;  // NB - tail: whole RBW groups
  return (NB - tail) / kLmHeadRBW + tail;
}

hipError_t launch_lm_head_argmax(const void* w, int V, int K, const void* x, int M, int ldx, float* logits,
                                 int logits_bf16, long long* out_idx, void* workspace,
                                 const void* norm_w, float eps, hipStream_t stream) {
  const int KT = K / kTileK;
  const int P = lm_head_partials(V);
  auto* status = static_cast<unsigned*>(workspace);
  auto* partials = reinterpret_cast<ArgmaxPartial*>(static_cast<unsigned char*>(workspace) + kLmHeadStatusBytes);
  const auto* nw = static_cast<const __bf16*>(norm_w);
  auto staged = [&](auto tag) {
    constexpr int kNC = decltype(tag)::value;
    if (nw != nullptr) {
      const size_t lds = (size_t)kLmHeadWaves * rms_wave_bytes(10, kNC, M, kLmHeadRBW);
      launch_kernel(lm_head_kernel<kLmHeadWaves, kLmHeadRBW, 10, kNC, true>, dim3(P + M), dim3(kLmHeadWaves * 64), lds, stream,
          static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, logits, V, logits_bf16, partials, status, out_idx, M,
          KT, nw, eps);
    } else {
      const size_t lds = (size_t)kLmHeadWaves * staged_wave_bytes(10, M, kLmHeadRBW);
      launch_kernel(lm_head_kernel<kLmHeadWaves, kLmHeadRBW, 10, kNC>, dim3(P + M), dim3(kLmHeadWaves * 64), lds, stream,
          static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, logits, V, logits_bf16, partials, status, out_idx, M,
          KT, nullptr, 0.f);
    }
  };
  // K/32 = 80: 8 waves x 10 k-tiles; for M <= 8 the activations are staged
  // through LDS (the wave's 40 M chunks over 64 lanes).
  if (KT == 80 && M <= 8) {
    switch ((40 * M + 63) / 64) {
      case 1:
        staged(std::integral_constant<int, 1>{});
        break;
      case 2:
        staged(std::integral_constant<int, 2>{});
        break;
      case 3:
        staged(std::integral_constant<int, 3>{});
        break;
      case 4:
        staged(std::integral_constant<int, 4>{});
        break;
      default:
        staged(std::integral_constant<int, 5>{});
        break;
    }
  } else if (nw != nullptr) {
    return hipErrorInvalidValue;  // the fused RMSNorm serves K = 2560, M <= 8 (checked by the caller)
  } else if (KT == 80) {
    launch_kernel(lm_head_kernel<kLmHeadWaves, kLmHeadRBW, 10>, dim3(P + M), dim3(kLmHeadWaves * 64), 0, stream,
        static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, logits, V, logits_bf16, partials, status, out_idx, M,
        KT, nullptr, 0.f);
  } else {
    launch_kernel(lm_head_kernel<kLmHeadWaves, kLmHeadRBW, 0>, dim3(P + M), dim3(kLmHeadWaves * 64), 0, stream,
        static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, logits, V, logits_bf16, partials, status, out_idx, M,
        KT, nullptr, 0.f);
  }
  return hipGetLastError();
}

}  // namespace lsk
