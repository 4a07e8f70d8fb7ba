// Projections of more than 16 rows on gfx950 MFMA:
// y[M][N] = epilogue(x[M][K] . W[N][K]^T), W in LSK_LAYOUT_MFMA16X32 (or its
// gate/up-interleaved form), bf16 in and out, fp32 accumulation.  Three
// kernels; launch_gemm_linear at the end of this file picks one:
//
//  * wdx::gemm_wdx_kernel, the prefill GEMM proper (M > 128, N a multiple of
//    128 or 192, K of 128: every Qwen3-4B projection).  256 tokens x 256, 192
//    or 128 weight rows x 64 K per stage and workgroup on
//    v_mfma_f32_32x32x16_bf16: weight fragments from HBM/L2 straight into
//    registers one stage ahead, activations DMA'd into a three-buffer LDS ring
//    two stages ahead, a counted stage barrier, the epilogue through LDS in
//    row order, and, with a workspace, the last partial round split along K
//    over the idle CUs ("Split-K of the last round" below).
//  * big::gemm256_kernel, 256 x 256 blocks with both operands staged in LDS,
//    for the M > 128 shapes with N a multiple of 256 that the wdx kernel does
//    not take (K an odd multiple of 64).
//  * gemm_linear_kernel, 128 x 128 blocks for the rest of the 128-row grid
//    (65..128 rows of N >= 8192, or N a multiple of 128 with K an odd
//    multiple of 64 that the 256 x 256 kernel cannot take).  Each packed 1 KB weight
//    tile already is a v_mfma_f32_16x16x32_bf16 operand in lane order, so the
//    weight half of every LDS stage is a straight linear copy; the activation
//    half is re-tiled into the same operand order as it is copied, so both
//    operands are read with linear 16-byte LDS loads.  4 wavefronts in a 2x2
//    arrangement, each owning 64x64 = 4x4 MFMA tiles; LDS double buffered.
//
// Every kernel remaps workgroups so that each XCD walks a contiguous run of a
// grouped (token block, weight block) order whose resident window shares its
// weight and activation slices through the XCD's L2.  Rows of M <= 16 and
// shapes off the 128-row grid go to the decode kernels (decode.hip).
//
// Reference arithmetic replaced: F.linear at
// src/leanstack/runtime/qwen_explicit.py:748, :819, :828, :830, :1202-1208 and
// the cuTile GEMM of experiments/cutile/qwen_bf16_hot_kernels.py:24-36.

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <type_traits>
#include <vector>

#include "lsk_internal.h"

namespace lsk {
namespace {

// Polls of a split block's arrival word before a split-K wait gives up
// (set_linear_wait_limit).
std::atomic<unsigned> g_wait_limit{kSkSpinLimit};

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRbPerBlock = kGemmBN / kTileRows;     // 8 weight row-blocks
constexpr int kMbPerBlock = kGemmBM / kTileRows;     // 8 token blocks of 16
constexpr int kKtPerStage = kGemmBK / kTileK;        // 2 K tiles per stage
constexpr int kWTiles = kRbPerBlock * kKtPerStage;   // 16
constexpr int kXTiles = kMbPerBlock * kKtPerStage;   // 16
constexpr int kStageTiles = kWTiles + kXTiles;       // 32 x 1 KB
constexpr int kLoadsPerThread = kStageTiles / kWaves;  // 8 (4 weight + 4 activation)

// Activation chunk of row `row`; the load is unconditional so the main loop
// has no branches that would split the accumulators' live ranges.  Rows past
// M are clamped to row M-1 instead of zeroed: output row m depends on
// activation row m only, and rows >= M are never stored, so the duplicate data
// is harmless.  No mask means no use of the loaded value at load time, which
// would force a vmcnt wait right after issue and expose the load latency.
__device__ __forceinline__ bf16x8_t load_x_row(const __bf16* __restrict__ x, int ldx, int M, int row, int k) {
  const int r = row < M ? row : M - 1;
  return *reinterpret_cast<const bf16x8_t*>(x + (size_t)r * ldx + k);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Block order.  Workgroup b runs on XCD b % 8 (round-robin dispatch), so each
// XCD gets a contiguous run of the logical order; inside it, tiles go in
// groups of kGroupM token blocks, all weight blocks of a group before the next
// group, token-block fastest.  The ~32 workgroups resident on one XCD at a
// time then cover about kGroupM token blocks x 32/kGroupM weight blocks, so
// their weight and activation slices are shared through that XCD's L2
// instead of the whole activation matrix being re-streamed per weight block.
constexpr int kGroupM = 8;

__device__ __forceinline__ void block_coords(int n_blocks, int m_blocks, int& nb, int& mb) {
  const int total = n_blocks * m_blocks;
  int logical = blockIdx.x;
  if (total % 8 == 0) logical = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
  const int group = logical / (kGroupM * n_blocks);
  const int first_m = group * kGroupM;
  const int group_m = min(m_blocks - first_m, kGroupM);
  const int in_group = logical - group * kGroupM * n_blocks;
  mb = first_m + in_group % group_m;
  nb = in_group / group_m;
}

struct StageRegs {
  bf16x8_t v[kLoadsPerThread];
};

// Global loads of one K stage into registers.  Thread (wave, lane) copies
// lane slot `lane` of tiles wave*4 .. wave*4+3 of both halves.
__device__ __forceinline__ void load_stage(StageRegs& r, const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x,
                                           int ldx, int M, int KT, int rb_base, int m_base, int kt0, int wave,
                                           int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = wave * 4 + j;
    const int rb = rb_base + t / kKtPerStage;
    const int kt = kt0 + t % kKtPerStage;
    r.v[j] = w[((size_t)rb * KT + kt) * 64 + lane];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = wave * 4 + j;
    const int row = m_base + (t / kKtPerStage) * 16 + (lane & 15);
    const int k = (kt0 + t % kKtPerStage) * kTileK + 8 * (lane >> 4);
    r.v[4 + j] = load_x_row(x, ldx, M, row, k);
  }
}

__device__ __forceinline__ void store_stage(bf16x8_t (*lds)[64], const StageRegs& r, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) lds[wave * 4 + j][lane] = r.v[j];
#pragma unroll
  for (int j = 0; j < 4; ++j) lds[kWTiles + wave * 4 + j][lane] = r.v[4 + j];
}

template <int EPI>
__global__ __launch_bounds__(kThreads) void gemm_linear_kernel(const bf16x8_t* __restrict__ w,
                                                               const __bf16* __restrict__ x, int ldx,
                                                               __bf16* __restrict__ y, int ldy,
                                                               const __bf16* __restrict__ residual, int ldr,
                                                               int M, int KT, int n_blocks, int m_blocks) {
  __shared__ bf16x8_t lds[2][kStageTiles][64];

  int nb, mb;
  block_coords(n_blocks, m_blocks, nb, mb);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave & 1;   // weight-row half of the block
  const int wm = wave >> 1;  // token half of the block
  const int rb_base = nb * kRbPerBlock;
  const int m_base = mb * kGemmBM;

  f32x4_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int stages = KT / kKtPerStage;
  StageRegs regs;
  load_stage(regs, w, x, ldx, M, KT, rb_base, m_base, 0, wave, lane);
  store_stage(lds[0], regs, wave, lane);
  __syncthreads();

  auto compute = [&](int cur) {
#pragma unroll
    for (int kk = 0; kk < kKtPerStage; ++kk) {
      bf16x8_t wf[4], xf[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) wf[a] = lds[cur][(wn * 4 + a) * kKtPerStage + kk][lane];
#pragma unroll
      for (int b = 0; b < 4; ++b) xf[b] = lds[cur][kWTiles + (wm * 4 + b) * kKtPerStage + kk][lane];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma16(wf[a], xf[b], acc[a][b]);
    }
  };
  for (int s = 0; s + 1 < stages; ++s) {
    load_stage(regs, w, x, ldx, M, KT, rb_base, m_base, (s + 1) * kKtPerStage, wave, lane);
    __builtin_amdgcn_sched_barrier(0);
    compute(s & 1);
    store_stage(lds[(s + 1) & 1], regs, wave, lane);
    __syncthreads();
  }
  compute((stages - 1) & 1);

  // Lane (g, c) of tile (a, b) holds rows 4g..4g+3 of weight row-block a
  // for token c of token block b.
  const int g = lane >> 4;
  const int c = lane & 15;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int m = m_base + (wm * 4 + b) * 16 + c;
    if (m >= M) continue;
    if constexpr (EPI == static_cast<int>(Epilogue::kSiluMul)) {
#pragma unroll
      for (int a = 0; a < 4; a += 2) {
        const int pair = (rb_base + wn * 4 + a) / 2;
        const int j = pair * 16 + 4 * g;
        unsigned short o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = bf16_bits(silu_mul_bf16(acc[a][b][i], acc[a + 1][b][i]));
        *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + j) =
            u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
      }
    } else {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int n = (rb_base + wn * 4 + a) * 16 + 4 * g;
        unsigned short o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = bf16_round(acc[a][b][i]);
          if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd))
            v = static_cast<float>(residual[(size_t)m * ldr + n + i]) + v;
          o[i] = bf16_bits(v);
        }
        *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + n) =
            u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large-tile variant: 256 (weight rows) x 256 (tokens) x 64 (K) blocks, four
// waves each owning a 128 x 128 tile of v_mfma_f32_32x32x16_bf16 (the full-
// rate MFMA on gfx950; the 16x16x32 form issues at about half its rate).  A
// 128 x 128 wave tile reads 8 KB of operands from LDS per 64 MFMAs, half the
// LDS bandwidth at peak MFMA rate, where the 64 x 64 tiles above need all of
// it.  Accumulators (256 per lane) live in the accumulation registers.
//
// Weight operand: a 32-row x 16-K A fragment is assembled from two packed
// 16 x 32 tiles by lane remapping (rows 0-15 from tile 2a, 16-31 from 2a+1),
// so the weights still arrive in LDS by a linear 1 KB copy per tile.  For the
// gate/up layout that pairing puts gate rows 0-15 and up rows 16-31 of the
// same 16 intermediate outputs in the same lane (accumulator j and j + 8).
// Activation operand: 32 tokens x 16 K fragments in B-operand lane order,
// with an XOR swizzle on the token slot so that both the coalesced global
// reads (8 lanes per 128-byte row) and the fragment reads hit 16 distinct
// bank groups per 16-lane pass.
namespace big {

constexpr int BN = 256, BM = 256, BK = 64;
constexpr int kThreads = 256;
constexpr int kWBytes = BN * BK * 2;                // 32 KB of weight tiles per stage
constexpr int kStageBytes = kWBytes + BM * BK * 2;  // + 32 KB of activation fragments
constexpr int kChunks = 8;                          // 16-byte chunks per thread per half-stage

typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// LDS byte offset of activation chunk (token m of the block, 8-wide K group k8 of the stage).
__device__ __forceinline__ int x_lds_off(int m, int k8) {
  return kWBytes + ((m >> 5) * 4 + (k8 >> 1)) * 1024 + ((((m & 31) ^ (2 * k8)) + 32 * (k8 & 1)) << 4);
}

struct Regs {
  bf16x8_t w[kChunks];
  bf16x8_t x[kChunks];
};

__device__ __forceinline__ void load_w(Regs& r, const bf16x8_t* __restrict__ w, int KT, int rb0, int s, int tid) {
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int u = c * kThreads + tid;
    const int tile = u >> 6;  // 32 tiles: (row-block, k-tile) = (tile / 2, tile % 2)
    r.w[c] = w[((size_t)(rb0 + (tile >> 1)) * KT + 2 * s + (tile & 1)) * 64 + (u & 63)];
  }
}

__device__ __forceinline__ void load_x(Regs& r, const __bf16* __restrict__ x, int ldx, int M, int m0, int s,
                                       int tid) {
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int u = c * kThreads + tid;
    r.x[c] = load_x_row(x, ldx, M, m0 + (u >> 3), s * BK + (u & 7) * 8);
  }
}

__device__ __forceinline__ void store_stage(unsigned char* buf, const Regs& r, int tid) {
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int u = c * kThreads + tid;
    *reinterpret_cast<bf16x8_t*>(buf + u * 16) = r.w[c];
  }
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int u = c * kThreads + tid;
    *reinterpret_cast<bf16x8_t*>(buf + x_lds_off(u >> 3, u & 7)) = r.x[c];
  }
}

// Instruction-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100, kSchedDsWrite = 0x200;

template <int EPI>
__global__ __launch_bounds__(kThreads, 1) void gemm256_kernel(const bf16x8_t* __restrict__ w,
                                                              const __bf16* __restrict__ x, int ldx,
                                                              __bf16* __restrict__ y, int ldy,
                                                              const __bf16* __restrict__ residual, int ldr, int M,
                                                              int KT, int n_blocks, int m_blocks) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kStageBytes];

  int nb, mb;
  block_coords(n_blocks, m_blocks, nb, mb);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int rb0 = nb * (BN / kTileRows);
  const int m0 = mb * BM;

  // Per-lane fragment offsets inside a stage.  Weight A fragment for n-tile
  // `an` (32 rows) and 16-K step q: rows from tiles 2an / 2an+1.
  const int li = lane & 31;
  const int kg = lane >> 5;
  const int w_lane = (li >> 4) * 2048 + kg * 256 + (li & 15) * 16;
  int x_lane[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) x_lane[q] = kWBytes + q * 1024 + ((((li) ^ (4 * q + 2 * kg)) + 32 * kg) << 4);

  f32x16_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;

  // Fragments of one 16-K step: four 32-row weight tiles, four 32-token activation tiles.
  auto read_frags = [&](bf16x8_t* fa, bf16x8_t* fb, const unsigned char* buf, int q) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
      fa[a] = *reinterpret_cast<const bf16x8_t*>(buf + (wn * 4 + a) * 4096 + q * 512 + w_lane);
#pragma unroll
    for (int b = 0; b < 4; ++b) fb[b] = *reinterpret_cast<const bf16x8_t*>(buf + (wm * 4 + b) * 4096 + x_lane[q]);
  };
  auto mfma_step = [&](const bf16x8_t* fa, const bf16x8_t* fb) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = mfma32(fa[a], fb[b], acc[a][b]);
  };

  // Software pipeline over 64-K stages with two LDS buffers.  While the MFMAs
  // of stage s run on buffer s&1, the same instruction stream (i) reads the
  // fragments of the next 16-K step into the idle register set, (ii) writes
  // stage s+1 from registers into buffer (s+1)&1 and (iii) issues the global
  // loads of stage s+2.  One barrier per stage, before the last 16-K step,
  // publishes buffer (s+1)&1 and retires every read of buffer s&1.  Stage
  // indices past the end are clamped: the redundant loads stay in bounds and
  // the data they stage is never multiplied.
  const int stages = KT / 2;
  Regs regs;
  load_w(regs, w, KT, rb0, 0, tid);
  load_x(regs, x, ldx, M, m0, 0, tid);
  store_stage(lds, regs, tid);
  const int s1 = min(1, stages - 1);
  load_w(regs, w, KT, rb0, s1, tid);
  load_x(regs, x, ldx, M, m0, s1, tid);
  __syncthreads();

  bf16x8_t fa0[4], fb0[4], fa1[4], fb1[4];
  read_frags(fa0, fb0, lds, 0);
  for (int s = 0; s < stages; ++s) {
    const unsigned char* cur = lds + (s & 1) * kStageBytes;
    unsigned char* nxt = lds + ((s + 1) & 1) * kStageBytes;
    const int ls = min(s + 2, stages - 1);

    read_frags(fa1, fb1, cur, 1);
    mfma_step(fa0, fb0);
    store_stage(nxt, regs, tid);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsWrite, 2, 0);
    }

    read_frags(fa0, fb0, cur, 2);
    load_w(regs, w, KT, rb0, ls, tid);
    mfma_step(fa1, fb1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8, 0);

    read_frags(fa1, fb1, cur, 3);
    load_x(regs, x, ldx, M, m0, ls, tid);
    mfma_step(fa0, fb0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8, 0);

    __syncthreads();
    read_frags(fa0, fb0, nxt, 0);
    mfma_step(fa1, fb1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8, 0);
  }

  // Lane l of tile (a, b) holds D[8*(j/4) + 4*(l/32) + j%4][l%32], j = 0..15.
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int m = m0 + (wm * 4 + b) * 32 + li;
    if (m >= M) continue;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int an = nb * 8 + wn * 4 + a;  // global 32-row tile index
      if constexpr (EPI == static_cast<int>(Epilogue::kSiluMul)) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int n = an * 16 + 8 * jj + 4 * kg;  // intermediate column
          unsigned short o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = bf16_bits(silu_mul_bf16(acc[a][b][4 * jj + e], acc[a][b][4 * jj + 8 + e]));
          *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + n) =
              u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
        }
      } else {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int n = an * 32 + 8 * jj + 4 * kg;
          unsigned short o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = bf16_round(acc[a][b][4 * jj + e]);
            if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd))
              v = static_cast<float>(residual[(size_t)m * ldr + n + e]) + v;
            o[e] = bf16_bits(v);
          }
          *reinterpret_cast<u32x2_t*>(y + (size_t)m * ldy + n) =
              u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
        }
      }
    }
  }
}

template <int EPI>
hipError_t launch(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                  const void* residual, int ldr, hipStream_t stream) {
  const int n_blocks = N / BN;
  const int m_blocks = (M + BM - 1) / BM;
  launch_kernel(gemm256_kernel<EPI>, dim3(n_blocks * m_blocks), dim3(kThreads), 0, stream,
      static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, static_cast<__bf16*>(y), ldy,
      static_cast<const __bf16*>(residual), ldr, M, K / kTileK, n_blocks, m_blocks);
  return hipGetLastError();
}

}  // namespace big

// Weights-direct variant of the 256x256x64 kernel (and of 192x256x64 and
// 128x256x64 ones, chosen by choose_tiles).  Each wave loads its own weight fragments from
// global memory straight into registers: a packed 1 KB tile already is MFMA
// operand data in lane order, so a 32-row A fragment is two 512-byte
// contiguous runs and needs no LDS staging.  Only the activations go
// through LDS, and they go there by DMA (buffer_load ... lds): no VGPRs and
// no ds_write instructions.  With 256-row blocks each wave owns 64 weight
// rows over all 256 tokens, so every weight line is fetched once per
// workgroup (32 KB of weights, 32 KB of activations per stage and CU through
// the texture path, 128 KB of LDS fragment reads), with 128-row blocks 32
// rows the same way; the 192-row blocks keep two waves across N and two across tokens, and
// there the two waves that share a weight-row half fetch the same lines, the
// second mostly from L1.
// Weight fragments are prefetched one stage ahead into the idle one of two
// register sets, activations two stages ahead into the free one of three
// LDS buffers; the stage loop is unrolled by six so both rotations run
// without copies, which requires an even number of stages.
namespace wdx {

constexpr int BN = 256, BM = 256, BK = 64;
// Wave tile: A 32-row weight tiles x TB 32-token tiles.  The 4 waves of a
// workgroup are TB/2 across N and 8/TB across the 256 tokens, so a block
// has 16*A*TB weight rows.  Built: (A, TB) = (2, 8) -> 256 rows, every wave
// over all tokens; (3, 4) -> 192 rows (QKV at 2048 tokens: 256 blocks in
// one round instead of 192 blocks of 256 rows); (1, 8) -> 128 rows, every
// wave over all tokens (small token counts, see choose_tiles).
template <int A, int TB>
constexpr int kBN = 16 * A * TB;
constexpr int kRowsWide = kBN<2, 8>;  // 256
constexpr int kRows192 = kBN<3, 4>;
constexpr int kRows128 = kBN<1, 8>;   // every wave 32 rows over all 256 tokens
constexpr int kThreads = 256;
constexpr int kXStageBytes = BM * BK * 2;  // 32 KB of activation fragments per stage

using big::f32x16_t;
using big::mfma32;
using big::kSchedMfma;
using big::kSchedVmemRead;
using big::kSchedDsRead;

template <int A>
struct WFrags {
  bf16x8_t v[4][A];  // [16-K step q][32-row tile a]
};

// A fragment (32 rows x 16 K) of tile a, step q: lane (li, kg) takes row li of
// the two 16-row packed tiles 2a, 2a+1 and K chunk 2(q&1)+kg of k-tile q/2.
template <int A>
__device__ __forceinline__ void load_w(WFrags<A>& f, const bf16x8_t* __restrict__ wl, int KT, int s) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int a = 0; a < A; ++a) f.v[q][a] = wl[((size_t)(2 * a) * KT + 2 * s + (q >> 1)) * 64 + (q & 1) * 32];
}

struct Args {
  const bf16x8_t* w;
  const __bf16* x;
  __bf16* y;
  const __bf16* residual;
  int ldx, ldy, ldr, M, KT, n_blocks, m_blocks;
  int wide_io;  // y (and the residual) allow 16-byte row accesses
};

typedef __attribute__((address_space(3))) void lds_void_t;

// Activation stage s of block rows m0.. straight into LDS: 256 tokens x 64 K
// as 128-byte rows, token t's 16-byte chunk c at position c ^ f(t) with
// f(t) = (t ^ (t >> 3)) & 7.  The B-fragment reads (lane li reads one chunk
// of token li) then hit distinct banks for any 8 consecutive lanes within
// a 128-byte bank row and for any 16 within a 256-byte one.  One
// buffer_load_dwordx4 ... lds moves 1 KB = 8 rows (block j = tokens 8j..):
// lane l lands at row r = l >> 3, position l & 7, so it fetches chunk
// (l & 7) ^ r ^ (j & 7) of its row; the 8 lanes of a row still read one
// whole 128-byte line.  Rows past the last token re-read it (rmax); the
// buffer covers exactly the block's rows.
// MUBUF, not FLAT: a FLAT load that writes LDS makes the compiler drain
// every counter before the next dependent use.
__device__ __forceinline__ void dma_x(unsigned char* buf, __amdgpu_buffer_rsrc_t rsrc, int ldx, int rmax, int s,
                                      int wave, int lane) {
  const int r = lane >> 3;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int j = wave * 8 + i;  // 1 KB block: tokens 8j .. 8j+7 (j & 7 == i)
    const int c = (lane & 7) ^ r ^ i;
    const int row = min(8 * j + r, rmax);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(buf + j * 1024), 16, (row * ldx + c * 8) * 2,
                                             s * BK * 2, 0, 0);
  }
}

// The stage barrier: s_waitcnt vmcnt(4A + 8) lgkmcnt(0), then s_barrier.
// Only the current stage's 4A weight loads and 8 activation DMAs may still
// be in flight after it, so the previous stage's DMA has landed in every
// wave.  Not __syncthreads: its release fence waits for vmcnt(0), i.e. for
// the loads just issued too.  The builtins (not inline asm) let the
// compiler's wait-counter model see these waits; the empty asm statements
// keep memory accesses from moving across them.
template <int A>
__device__ __forceinline__ void stage_sync() {
  constexpr int vm = 4 * A + 8;
  constexpr int imm = (vm & 15) | ((vm >> 4) << 14) | (7 << 4);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(imm);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// acc[a][b] += W rows of 32-row tiles (wn*A + a) x tokens of 32-token tiles
// (wm*TB + b) over stages [s0, s1) (s1 - s0 even) of block (nb, mb).
//
// Software pipeline over 64-K stages with three LDS activation buffers.
// While the MFMAs of stage s run on buffer cur with weight fragments wc, the
// same instruction stream reads the activation fragments of the next 16-K
// step, loads stage s+1's weight fragments into the idle register set and
// DMAs stage s+2's activations into the buffer stage s-1 read.  The barrier
// before the last 16-K step publishes stage s+1's buffer (its DMA was issued
// one stage earlier) and retires every read of this stage's.  Stage indices
// past s1 are clamped: those loads stay in bounds and the data they stage is
// never multiplied.
template <int kM, int ND, int VO, int NV>
__device__ __forceinline__ void sched_step() {
  // kM MFMAs of one 16-K step, each followed by one of the step's ND LDS
  // reads (the first ND) and one of its NV global loads (MFMAs VO..VO+NV-1).
#pragma unroll
  for (int i = 0; i < kM; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    if (i < ND) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    if (i >= VO && i < VO + NV) __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
  }
}

template <int A, int TB>
__device__ __forceinline__ void mainloop(f32x16_t (&acc)[A][TB], const Args& g, unsigned char* xa, unsigned char* xb,
                                         unsigned char* xc, int nb, int mb, int s0, int s1) {
  constexpr int WN = TB / 2;  // waves across N
  // Opaque per call: keeps the per-lane offsets below from being hoisted out
  // of a caller's loop over blocks, where they would stay live (and spill)
  // across the epilogues.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave % WN;
  const int wm = wave / WN;
  const int m0 = mb * BM;
  const int li = lane & 31;
  const int kg = lane >> 5;
  const int KT = g.KT;
  const int rmax = min(g.M - m0, BM) - 1;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.x + (size_t)m0 * g.ldx), (short)0, (int)((unsigned)(rmax + 1) * (unsigned)g.ldx * 2u), 0x00020000);

  // This lane's element of weight fragment (a=0, q=0) at stage 0.
  const bf16x8_t* wl =
      g.w + ((size_t)(nb * (kBN<A, TB> / kTileRows) + wn * 2 * A + (li >> 4)) * KT) * 64 + (li & 15) + kg * 16;
  // Chunk 2q + kg of token t = wm*TB*32 + b*32 + li sits at position
  // (2q + kg) ^ (li & 7) ^ (li >> 3) ^ 4(b & 1): x_lane[q] holds it for
  // even b, odd b flip bit 6 of the byte offset.
  int x_lane[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    x_lane[q] = wm * TB * 4096 + li * 128 + ((((2 * q + kg) ^ (li & 7) ^ (li >> 3))) << 4);

  auto read_b = [&](bf16x8_t* fb, const unsigned char* buf, int q) {
#pragma unroll
    for (int b = 0; b < TB; ++b)
      fb[b] = *reinterpret_cast<const bf16x8_t*>(buf + b * 4096 + (x_lane[q] ^ ((b & 1) << 6)));
  };
  auto mfma_step = [&](const bf16x8_t* fa, const bf16x8_t* fb) {
#pragma unroll
    for (int a = 0; a < A; ++a)
#pragma unroll
      for (int b = 0; b < TB; ++b) acc[a][b] = mfma32(fa[a], fb[b], acc[a][b]);
  };

  WFrags<A> wf0, wf1;
  bf16x8_t fb0[TB], fb1[TB];

  // Interleave groups per 16-K step: A*TB MFMAs with the step's TB LDS
  // reads and its global traffic (4A weight loads in step 0, 8 DMA in
  // step 1).
  constexpr int kM = A * TB;
  // Step 1's 8 DMAs go after the MFMAs that follow its TB LDS reads, as far
  // as the step has MFMAs there: for A = 1 (kM = TB = 8) from the first one.
  constexpr int kDmaSlot = kM - 8 >= TB ? TB : (kM > 8 ? kM - 8 : 0);
  // Stage s multiplies buffer cur, DMAs the activations of stage s + 2 into
  // dst (the buffer stage s - 1 read) and, before its barrier, waits for the
  // DMA of stage s + 1 (issued one stage earlier; only the 4A weight loads
  // and 8 DMA of this stage may still be in flight).
  auto stage = [&](int s, const WFrags<A>& wc, WFrags<A>& wn_, const unsigned char* cur, unsigned char* dst,
                   const unsigned char* nxt) {
    const int sw = min(s + 1, s1 - 1);
    const int sx = min(s + 2, s1 - 1);

    __builtin_amdgcn_sched_barrier(0);
    read_b(fb1, cur, 1);
    load_w(wn_, wl, KT, sw);
    mfma_step(wc.v[0], fb0);
    sched_step<kM, TB, 0, 4 * A>();

    __builtin_amdgcn_sched_barrier(0);
    read_b(fb0, cur, 2);
    dma_x(dst, xr, g.ldx, rmax, sx, wave, lane);
    mfma_step(wc.v[1], fb1);
    sched_step<kM, TB, kDmaSlot, 8>();

    __builtin_amdgcn_sched_barrier(0);
    read_b(fb1, cur, 3);
    mfma_step(wc.v[2], fb0);
    sched_step<kM, TB, 0, 0>();

    // Publishes nxt (stage s + 1's DMA) and retires every read of cur.
    stage_sync<A>();
    read_b(fb0, nxt, 0);
    mfma_step(wc.v[3], fb1);
    sched_step<kM, TB, 0, 0>();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Every wave is past its last read of the buffers (a previous call's
  // stages) before the prologue overwrites xa and xb.
  __syncthreads();
  dma_x(xa, xr, g.ldx, rmax, s0, wave, lane);
  dma_x(xb, xr, g.ldx, rmax, min(s0 + 1, s1 - 1), wave, lane);
  load_w(wf0, wl, KT, s0);
  stage_sync<A>();
  read_b(fb0, xa, 0);
  int s = s0;
  for (; s + 6 <= s1; s += 6) {
    stage(s, wf0, wf1, xa, xc, xb);
    stage(s + 1, wf1, wf0, xb, xa, xc);
    stage(s + 2, wf0, wf1, xc, xb, xa);
    stage(s + 3, wf1, wf0, xa, xc, xb);
    stage(s + 4, wf0, wf1, xb, xa, xc);
    stage(s + 5, wf1, wf0, xc, xb, xa);
  }
  if (s + 2 <= s1) {
    stage(s, wf0, wf1, xa, xc, xb);
    stage(s + 1, wf1, wf0, xb, xa, xc);
    if (s + 4 <= s1) {
      stage(s + 2, wf0, wf1, xc, xb, xa);
      stage(s + 3, wf1, wf0, xa, xc, xb);
    }
  }
}

// Epilogue of this lane's 32x32 tile (a, b) of block (nb, mb).  src(p)
// returns elements 2p, 2p+1 of the lane's 16 fp32 results of the tile.
// Lane l of tile (a, b) holds D[8*(j/4) + 4*(l/32) + j%4][l%32], j = 0..15.
template <int EPI, int A, int TB, typename Src>
__device__ __forceinline__ void store_one_tile(Src src, const Args& g, int nb, int mb, int a, int b) {
  constexpr int WN = TB / 2;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % WN;
  const int wm = wave / WN;
  const int li = lane & 31;
  const int kg = lane >> 5;
  const int m = mb * BM + (wm * TB + b) * 32 + li;
  if (m >= g.M) return;
  const int an = (nb * WN + wn) * A + a;  // global 32-row tile index
  if constexpr (EPI == static_cast<int>(Epilogue::kSiluMul)) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int n = an * 16 + 8 * jj + 4 * kg;  // intermediate column
      const float2 g0 = src(2 * jj), g1 = src(2 * jj + 1);
      const float2 u0 = src(2 * jj + 4), u1 = src(2 * jj + 5);
      const unsigned short o0 = bf16_bits(silu_mul_bf16(g0.x, u0.x));
      const unsigned short o1 = bf16_bits(silu_mul_bf16(g0.y, u0.y));
      const unsigned short o2 = bf16_bits(silu_mul_bf16(g1.x, u1.x));
      const unsigned short o3 = bf16_bits(silu_mul_bf16(g1.y, u1.y));
      *reinterpret_cast<u32x2_t*>(g.y + (size_t)m * g.ldy + n) =
          u32x2_t{o0 | ((unsigned)o1 << 16), o2 | ((unsigned)o3 << 16)};
    }
  } else {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int n = an * 32 + 8 * jj + 4 * kg;
      const float2 p0 = src(2 * jj), p1 = src(2 * jj + 1);
      float v[4] = {bf16_round(p0.x), bf16_round(p0.y), bf16_round(p1.x), bf16_round(p1.y)};
      if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = static_cast<float>(g.residual[(size_t)m * g.ldr + n + e]) + v[e];
      }
      *reinterpret_cast<u32x2_t*>(g.y + (size_t)m * g.ldy + n) =
          u32x2_t{bf16_bits(v[0]) | ((unsigned)bf16_bits(v[1]) << 16),
                  bf16_bits(v[2]) | ((unsigned)bf16_bits(v[3]) << 16)};
    }
  }
}

// Epilogue of the whole block straight from the accumulators.
template <int EPI, int A, int TB>
__device__ __forceinline__ void store_tile(const f32x16_t (&acc)[A][TB], const Args& g, int nb, int mb) {
#pragma unroll
  for (int b = 0; b < TB; ++b)
#pragma unroll
    for (int a = 0; a < A; ++a)
      store_one_tile<EPI, A, TB>([&](int p) { return make_float2(acc[a][b][2 * p], acc[a][b][2 * p + 1]); }, g, nb,
                                 mb, a, b);
}

// Epilogue of a whole block through LDS.  Stored straight from the
// accumulators (store_tile), each store instruction writes 8 bytes per lane
// into 32 different token rows; every CU does that at the same moment at
// the end of a round, and it cost 14-19 us of a 2048 x 8192 output.  Here
// each wave rounds its results to bf16 into its own 16 KB of the (free)
// activation buffers, token-major, then reads them back 16 bytes per lane
// in row order, so one store instruction covers whole row segments (8 rows
// of 128 bytes for the 2x8 wave tile).  Two passes of half the wave's
// tokens each.  Needs every wave past its last activation read and no DMA
// in flight (the caller's barrier).  Rounding is that of store_one_tile:
// bf16 products, then the residual added in fp32 and rounded again.
//
// Region layout: token row r of C bytes (C = 64A plain, 32A SiLU*up), its
// 16-byte chunk c at position c ^ (f(r) mod C/16), f(r) = (r ^ (r >> 3)) & 7
// (C/16 is 8, 4, 12 or 6: the XOR uses the low 3, 2, 2 or 1 bits so every
// position stays in the row).
template <int C>
__device__ __forceinline__ int epi_pos(int r, int c) {
  constexpr int kChunks = C / 16;
  constexpr int kMask = kChunks % 8 == 0 ? 7 : kChunks % 4 == 0 ? 3 : kChunks % 2 == 0 ? 1 : 0;
  return r * C + ((c ^ ((r ^ (r >> 3)) & kMask)) << 4);
}

template <int EPI, int A, int TB>
__device__ __forceinline__ void store_tile_lds(const f32x16_t (&acc)[A][TB], const Args& g, int nb, int mb,
                                               unsigned char* xa, unsigned char* xb) {
  constexpr int WN = TB / 2;
  constexpr bool kSilu = EPI == static_cast<int>(Epilogue::kSiluMul);
  constexpr int C = kSilu ? 32 * A : 64 * A;  // output bytes per token of this wave
  constexpr int HB = TB / 2;                  // token tiles per pass
  constexpr int kChunks = HB * 32 * C / 16;   // 16-byte chunks per pass
  static_assert(HB * 32 * C <= 16384, "a pass must fit the wave's 16 KB region");
  static_assert(kChunks % 64 == 0, "whole chunks per lane");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % WN;
  const int wm = wave / WN;
  const int li = lane & 31;
  const int kg = lane >> 5;
  unsigned char* reg = (wave < 2 ? xa : xb) + (wave & 1) * 16384;
  // First output column of this wave and its first token.
  const int n0 = (nb * WN + wn) * A * (kSilu ? 16 : 32);
  const int t0 = mb * BM + wm * TB * 32;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int b = 0; b < HB; ++b)
#pragma unroll
      for (int a = 0; a < A; ++a) {
        const f32x16_t& v = acc[a][h * HB + b];
        const int r = b * 32 + li;
        if constexpr (kSilu) {
          // rows 8jj + 4kg + e of the tile are gate, 16 + the same are up
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const int col = a * 16 + 8 * jj + 4 * kg;  // intermediate column within the wave
            unsigned short o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = bf16_bits(silu_mul_bf16(v[4 * jj + e], v[4 * jj + 8 + e]));
            *reinterpret_cast<u32x2_t*>(reg + epi_pos<C>(r, col >> 3) + (col & 7) * 2) =
                u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
          }
        } else {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int col = a * 32 + 8 * jj + 4 * kg;
            *reinterpret_cast<u32x2_t*>(reg + epi_pos<C>(r, col >> 3) + (col & 7) * 2) =
                u32x2_t{bf16_bits(v[4 * jj]) | ((unsigned)bf16_bits(v[4 * jj + 1]) << 16),
                        bf16_bits(v[4 * jj + 2]) | ((unsigned)bf16_bits(v[4 * jj + 3]) << 16)};
          }
        }
      }
    // The same wave reads back what it wrote: LDS executes one wave's
    // accesses in order.
#pragma unroll
    for (int i = 0; i < kChunks / 64; ++i) {
      const int k = i * 64 + lane;
      const int r = k / (C / 16);
      const int c = k % (C / 16);
      const int m = t0 + h * HB * 32 + r;
      const u32x4_t q = *reinterpret_cast<const u32x4_t*>(reg + epi_pos<C>(r, c));
      if (m >= g.M) continue;
      const int n = n0 + c * 8;
      __bf16* dst = g.y + (size_t)m * g.ldy + n;
      if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd)) {
        const __bf16* rs = g.residual + (size_t)m * g.ldr + n;
        u32x4_t rv;
        if (g.wide_io) {
          rv = *reinterpret_cast<const u32x4_t*>(rs);
        } else {
          const unsigned short* r16 = reinterpret_cast<const unsigned short*>(rs);
#pragma unroll
          for (int e = 0; e < 4; ++e) rv[e] = r16[2 * e] | ((unsigned)r16[2 * e + 1] << 16);
        }
        u32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = __builtin_bit_cast(float, q[e] << 16) + __builtin_bit_cast(float, rv[e] << 16);
          const float hi = __builtin_bit_cast(float, q[e] & 0xffff0000u) + __builtin_bit_cast(float, rv[e] & 0xffff0000u);
          o[e] = bf16_bits(lo) | ((unsigned)bf16_bits(hi) << 16);
        }
        if (g.wide_io) {
          *reinterpret_cast<u32x4_t*>(dst) = o;
        } else {
          reinterpret_cast<u32x2_t*>(dst)[0] = u32x2_t{o[0], o[1]};
          reinterpret_cast<u32x2_t*>(dst)[1] = u32x2_t{o[2], o[3]};
        }
      } else {
        if (g.wide_io) {
          *reinterpret_cast<u32x4_t*>(dst) = q;
        } else {
          reinterpret_cast<u32x2_t*>(dst)[0] = u32x2_t{q[0], q[1]};
          reinterpret_cast<u32x2_t*>(dst)[1] = u32x2_t{q[2], q[3]};
        }
      }
    }
  }
}

template <int A, int TB>
__device__ __forceinline__ void zero(f32x16_t (&acc)[A][TB]) {
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int b = 0; b < TB; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.f;
}

// ---- Split-K of the last round -------------------------------------------
//
// T output blocks on G CUs run ceil(T/G) rounds of whole-K blocks; when the
// last round is partial (R = T mod G blocks, or all T when T < G, e.g. 80
// blocks of the hidden-output projections at 2048 tokens) most CUs idle
// through it.  The launch therefore runs the first T - R blocks one per
// workgroup (the grouped, XCD-aware order of block_coords, so the ~32
// workgroups of an XCD share weight and activation lines in its L2) and
// splits each of the R last blocks into S = min(G / R, units / 4) chunks of
// 128-K units, all blocks' chunk s covering the same K range so that they
// share lines the same way.  The S workgroups of a split block each store
// their fp32 accumulators to a workspace slot and count themselves in the
// block's arrival word; once all S have arrived, workgroup s sums tiles
// [16s/S, 16(s+1)/S) of the block, its own partial first and then the other
// S - 1 slots in chunk order, and stores them with the epilogue, then counts itself out; the last one out
// clears both words.  R*S <= G, and whole-K blocks never wait, so every
// split workgroup gets a CU.  That holds only while no other kernel shares
// the device, so the waits are bounded: a workgroup that gives up (after
// Split::spin_limit polls) records it in the error word and stores NaN for
// its tiles instead of a partial sum, so a lost wait can never pass for a
// result.  The order
// of every sum is fixed by (T, G), so results are bitwise reproducible.
// Partials cross XCDs, whose L2s are not coherent with each other, so they
// are written and read with device-coherent (sc1) accesses, the ones
// agent-scope relaxed atomics use; no cache maintenance is needed.

typedef unsigned int u32x2v_t __attribute__((ext_vector_type(2)));
constexpr int kCoherent = 16;
constexpr unsigned kRawBufferDword3 = 0x00020000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t partial_rsrc(unsigned char* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, (int)kRawBufferDword3);
}

// Block t of the grouped order (kGroupM token blocks, all weight blocks of a
// group before the next group, token block fastest).
__device__ __forceinline__ void tile_coords(int t, int n_blocks, int m_blocks, int& nb, int& mb) {
  const int group = t / (kGroupM * n_blocks);
  const int first_m = group * kGroupM;
  const int group_m = min(m_blocks - first_m, kGroupM);
  const int in_group = t - group * kGroupM * n_blocks;
  mb = first_m + in_group % group_m;
  nb = in_group / group_m;
}

struct Split {
  unsigned* error;          // workspace word 0
  unsigned* flags;          // arrival, departure word per split block
  unsigned char* partials;  // kSkPartialBytes per split workgroup
  unsigned partial_bytes;   // R * S * kSkPartialBytes
  int dp;                   // blocks run whole (T - R)
  int R;                    // blocks split
  int S;                    // chunks per split block (1 = no split)
  int units;                // 128-K units per block (KT / 4)
  unsigned spin_limit;      // polls of the arrival word before a wait gives up
};

template <int EPI, int A, int TB>
__global__ __launch_bounds__(kThreads, 1) void gemm_wdx_kernel(Args g, Split k) {
  __shared__ __attribute__((aligned(1024))) unsigned char xa[kXStageBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char xb[kXStageBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char xc[kXStageBytes];
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  f32x16_t acc[A][TB];
  zero(acc);

  if (b < k.dp) {
    // Whole block; workgroup b runs on XCD b % 8, so give each XCD a
    // contiguous run of the grouped order.
    const int t = k.dp % 8 == 0 ? (b % 8) * (k.dp / 8) + b / 8 : b;
    int nb, mb;
    tile_coords(t, g.n_blocks, g.m_blocks, nb, mb);
    mainloop(acc, g, xa, xb, xc, nb, mb, 0, g.KT / 2);
    // The last stages' activation DMAs (clamped, never read) may still be
    // writing the buffers and other waves may still read them: both end
    // before the epilogue reuses them.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    store_tile_lds<EPI, A, TB>(acc, g, nb, mb, xa, xb);
    return;
  }
  // Chunk-major order: all split blocks' chunk 0, then chunk 1, ...
  const int r = b - k.dp;
  const int chunk = r / k.R;
  const int i = r % k.R;
  int nb, mb;
  if (k.dp == 0 && k.R % 8 == 0 && g.m_blocks % 2 == 0) {
    // Every block split (one partial round): workgroup r runs on XCD
    // i % 8, so give XCD x the contiguous run [x R/8, (x+1) R/8) of an
    // order grouped by token-block pairs; each XCD then covers a
    // rectangle (e.g. 5 weight blocks x 2 token blocks at 2048 tokens)
    // instead of every weight block of one token block.  down_proj at
    // 2048 tokens: 139 -> 134 us.  The map i -> (nb, mb) is one to one.
    const int i2 = (i % 8) * (k.R / 8) + i / 8;
    const int group = i2 / (2 * g.n_blocks);
    mb = group * 2 + i2 % 2;
    nb = (i2 - group * 2 * g.n_blocks) / 2;
  } else {
    tile_coords(k.dp + i, g.n_blocks, g.m_blocks, nb, mb);
  }
  const int u0 = chunk * k.units / k.S, u1 = (chunk + 1) * k.units / k.S;
  mainloop(acc, g, xa, xb, xc, nb, mb, 2 * u0, 2 * u1);

  // This workgroup sums tiles [ab0, ab1) of the block (each thread its own
  // quads of them); it keeps its partial of those in its accumulators and
  // publishes only the others.
  const int ab0 = chunk * A * TB / k.S, ab1 = (chunk + 1) * A * TB / k.S;
  // Publish this chunk's partial (slot chunk*R + i): quad q of tile (a, b)
  // of thread tid at ((4*(TB*a+b) + q) * 256 + tid) * 16 bytes, so each store
  // instruction writes 1 KB contiguously straight from four accumulators.
  const __amdgpu_buffer_rsrc_t parts = partial_rsrc(k.partials, k.partial_bytes);
  {
    const unsigned slot = (unsigned)r * (unsigned)kSkPartialBytes;
#pragma unroll
    for (int a = 0; a < A; ++a)
#pragma unroll
      for (int bb = 0; bb < TB; ++bb) {
        const int ab = a * TB + bb;
        if (ab >= ab0 && ab < ab1) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4_t v;
#pragma unroll
          for (int e = 0; e < 4; ++e) asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v[e]) : "a"(acc[a][bb][4 * q + e]));
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), parts, tid * 16,
                                                 slot + (ab * 4 + q) * kThreads * 16, kCoherent);
        }
      }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  unsigned* arrive = k.flags + 2 * i;
  unsigned* depart = arrive + 1;
  __shared__ int gave_up;
  if (tid == 0) {
    gave_up = 0;
    __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned spins = 0;
    while (__hip_atomic_load(arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)k.S) {
      if (spins++ >= k.spin_limit) {
        __hip_atomic_store(k.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gave_up = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
  const bool poison = gave_up != 0;

  // Sum this workgroup's share of the block's tiles over the S chunks: its
  // own chunk's partial (from its accumulators) first, then the other chunks
  // in chunk order, three chunks' loads in flight at a time (one round trip
  // per tile for S <= 4).  Loads past the last chunk put their offset beyond
  // the partials in the VGPR offset, which the buffer range check covers, and
  // return zeros without a memory access.
  const unsigned first = (unsigned)i * (unsigned)kSkPartialBytes;
  const unsigned chunk_stride = (unsigned)k.R * (unsigned)kSkPartialBytes;
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int bb = 0; bb < TB; ++bb) {
      const int ab = a * TB + bb;
      if (ab < ab0 || ab >= ab1) continue;
      f32x4_t sum[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(sum[q][e]) : "a"(acc[a][bb][4 * q + e]));
      for (int j0 = 0; j0 < k.S - 1; j0 += 3) {
        f32x4_t v[3][4];
#pragma unroll
        for (int g3 = 0; g3 < 3; ++g3) {
          const int j = j0 + g3;
          const int c = j < chunk ? j : j + 1;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const unsigned off = j < k.S - 1 ? first + c * chunk_stride + (ab * 4 + q) * kThreads * 16 : 0x80000000u;
            v[g3][q] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(parts, off + tid * 16, 0,
                                                                                          kCoherent));
          }
        }
#pragma unroll
        for (int g3 = 0; g3 < 3; ++g3)
#pragma unroll
          for (int q = 0; q < 4; ++q) sum[q] += v[g3][q];
      }
      if (poison) {
#pragma unroll
        for (int q = 0; q < 4; ++q) sum[q] = f32x4_t{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                                                     __builtin_nanf("")};
      }
      store_one_tile<EPI, A, TB>(
          [&](int p) { return make_float2(sum[p >> 1][2 * (p & 1)], sum[p >> 1][2 * (p & 1) + 1]); }, g, nb, mb, a,
          bb);
    }
  if (tid == 0 &&
      __hip_atomic_fetch_add(depart, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)k.S - 1) {
    __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(depart, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

inline Args make_args(int bn, const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                      const void* residual, int ldr) {
  Args g;
  g.w = static_cast<const bf16x8_t*>(w);
  g.x = static_cast<const __bf16*>(x);
  g.y = static_cast<__bf16*>(y);
  g.residual = static_cast<const __bf16*>(residual);
  g.ldx = ldx;
  g.ldy = ldy;
  g.ldr = ldr;
  g.M = M;
  g.KT = K / kTileK;
  g.n_blocks = N / bn;
  g.m_blocks = (M + BM - 1) / BM;
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  g.wide_io = a16(y) && ldy % 8 == 0 && (residual == nullptr || (a16(residual) && ldr % 8 == 0));
  return g;
}

// Blocks split and chunks per split block for T blocks of `units` 128-K
// units on `grid` CUs (R = 0 or S = 1: no split).  S = the most chunks the
// grid holds (at least 4 units each), rounded down to 4, 8 or 16 when it is
// 4 or more: each chunk's workgroup then sums an equal share of the block's
// 16 partial tiles.  Measured at M = 512 / 1024 (QKV S 5 -> 4: 42.6 -> 35.2
// us; down S 12 -> 8: 52.9 -> 45.2 us; o_proj S 6 -> 4: 45.1 -> 40.6 us).
inline void split_plan(int T, int units, int grid, int* R, int* S) {
  *R = grid > 0 ? T % grid : 0;
  *S = 1;
  if (*R == 0) return;
  int s = grid / *R;
  if (s > units / 4) s = units / 4;
  if (s > 16) s = 16;
  if (s >= 4) {
    while (s & (s - 1)) s &= s - 1;  // highest power of two <= s
  }
  if (s < 2) {
    *R = 0;
    return;
  }
  *S = s;
}

// Block height for an N x M problem on `grid` CUs, as the 32-row weight
// tiles per wave A of the wave tile: 3 = 192-row blocks when N allows them
// and they need fewer block-rows of work per CU than 256-row blocks (4;
// ceil(blocks / grid) rounds of BN rows each), e.g. QKV (N = 6144) at 2048
// tokens: 256 blocks of 192 rows in one round instead of 192 blocks of 256
// rows that leave a quarter of the CUs idle.  Ties keep 256.  Then 1 =
// 128-row blocks when that choice would split every block at least four
// ways over `split_grid` CUs (0: no split): half-height blocks halve each
// split workgroup's fp32 partial and need fewer chunks.  At 512 tokens:
// o_proj 29.5 -> 23.9 us, QKV 32.2 -> 28.9, down_proj 45.4 -> 41.2; where
// the blocks split fewer ways (every shape at 2048 tokens) or not at all
// (gate_up at 512) 128-row blocks measured slower.  Also 1 when the coarser
// plan splits two or three ways but 128-row blocks fit one round without a
// split and the measured costs favour them: per 64-K stage at full load a
// 128-row block takes about 0.85 us against 1.18 (192 rows) and 1.40 (256
// rows), and a split round adds about 0.06 us per block row for its partial
// exchange.  QKV at 768 and 1024 tokens 37.2 -> 32.6 and 41.1 -> 36.3 us,
// o_proj at 3072 66.1 -> 61.8; down_proj at 3072 (152 stages) keeps its
// split 256-row round.  And 1 whenever N is a multiple of 128 but of neither
// 192 nor 256 (e.g. the gate_up shard of 8-way tensor parallelism, 2432
// rows), which the 128 x 128 kernel would otherwise take.
inline int choose_tiles(int N, int m_blocks, int grid, int units, int split_grid) {
  if (N % kRowsWide != 0 && N % kRows192 != 0) return 1;  // N on the 128-row grid only
  int a = 4;
  if (N % kRows192 != 0) {
    a = 4;
  } else if (N % kRowsWide != 0) {
    a = 3;
  } else {
    const long r4 = ((long)(N / kRowsWide) * m_blocks + grid - 1) / grid;
    const long r3 = ((long)(N / kRows192) * m_blocks + grid - 1) / grid;
    a = r3 * kRows192 < r4 * kRowsWide ? 3 : 4;
  }
  if (split_grid > 0 && N % kRows128 == 0) {
    const int T = (N / (a == 3 ? kRows192 : kRowsWide)) * m_blocks;
    int R = 0, S = 1;
    split_plan(T, units, split_grid, &R, &S);
    if (T < split_grid && S >= 4) return 1;
    if (T < split_grid && S >= 2 && (N / kRows128) * m_blocks <= grid) {
      const int stages = 2 * units;
      const double t128 = 0.85 * stages;
      const double tc = (a == 3 ? 1.18 : 1.40) * ((stages + S - 1) / S) + 0.06 * (a == 3 ? kRows192 : kRowsWide);
      if (t128 < tc) return 1;
    }
  }
  return a;
}

// `grid` = CUs available to the split (0: no split, no workspace needed).
template <int EPI, int A, int TB>
hipError_t launch(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                  const void* residual, int ldr, void* workspace, int grid, hipStream_t stream) {
  const Args g = make_args(kBN<A, TB>, w, N, K, x, M, ldx, y, ldy, residual, ldr);
  const int T = g.n_blocks * g.m_blocks;
  Split k;
  k.units = g.KT / 4;
  split_plan(T, k.units, workspace != nullptr ? grid : 0, &k.R, &k.S);
  k.dp = T - k.R;
  auto* ws = static_cast<unsigned char*>(workspace);
  k.error = reinterpret_cast<unsigned*>(ws);
  k.flags = ws != nullptr ? reinterpret_cast<unsigned*>(ws + kSkFlagsOffset) : nullptr;
  k.partials = ws != nullptr ? ws + kSkPartialsOffset : nullptr;
  k.partial_bytes = (unsigned)((size_t)k.R * k.S * kSkPartialBytes);
  k.spin_limit = g_wait_limit.load(std::memory_order_relaxed);
  launch_kernel(gemm_wdx_kernel<EPI, A, TB>, dim3(k.dp + k.R * k.S), dim3(kThreads), 0, stream, g, k);
  return hipGetLastError();
}

}  // namespace wdx

template <int EPI>
hipError_t launch_cfg(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                      const void* residual, int ldr, hipStream_t stream) {
  const int n_blocks = N / kGemmBN;
  const int m_blocks = (M + kGemmBM - 1) / kGemmBM;
  launch_kernel(gemm_linear_kernel<EPI>, dim3(n_blocks * m_blocks), dim3(kThreads), 0, stream,
      static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, static_cast<__bf16*>(y), ldy,
      static_cast<const __bf16*>(residual), ldr, M, K / kTileK, n_blocks, m_blocks);
  return hipGetLastError();
}

}  // namespace

namespace {

bool sk_shape(int M, int N, int K) {
  return M > kGemmBM && (N % wdx::kRows128 == 0 || N % wdx::kRows192 == 0) && K % (2 * wdx::BK) == 0;
}

// Workgroups resident at once on `device` (the kernel holds 512 registers
// per lane, so one per CU), capped by the workspace's flag capacity: the
// split-K plan spreads the last round over this many.  Cached per device.
hipError_t sk_grid(int device, int* grid_out) {
  static std::mutex mu;
  static std::vector<int> cache;
  std::lock_guard<std::mutex> lock(mu);
  if (device >= (int)cache.size()) cache.resize(device + 1, 0);
  if (cache[device] == 0) {
    int cus = 0, per_cu = 0;
    hipError_t err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (err != hipSuccess) return err;
    err = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, reinterpret_cast<const void*>(&wdx::gemm_wdx_kernel<0, 2, 8>), wdx::kThreads, 0);
    if (err != hipSuccess) return err;
    int grid = cus * (per_cu > 0 ? per_cu : 1);
    cache[device] = grid < kSkMaxGrid ? grid : kSkMaxGrid;
  }
  *grid_out = cache[device];
  return hipSuccess;
}

}  // namespace

void set_linear_wait_limit(unsigned polls) { g_wait_limit.store(polls, std::memory_order_relaxed); }

size_t gemm_workspace_bytes(int device, int M, int N, int K, hipError_t* status) {
  *status = hipSuccess;
  if (!sk_shape(M, N, K)) return 0;
  int grid = 0;
  *status = sk_grid(device, &grid);
  if (*status != hipSuccess) return 0;
  return kSkPartialsOffset + (size_t)grid * kSkPartialBytes;
}

// The block GEMM's plan on the current device: `grid` = the CUs the last,
// partial round may split over (0 without a workspace, else every CU: both
// callers have checked that a workspace holds gemm_workspace_bytes) and the
// block height as choose_tiles returns it.  Shared by the launch and
// lsk_linear_plan.
static hipError_t wdx_plan(int M, int N, int K, bool has_ws, int* grid_out, int* tiles_out) {
  int device = 0, cus = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  err = sk_grid(device, &cus);
  if (err != hipSuccess) return err;
  const int grid = has_ws ? cus : 0;
  *grid_out = grid;
  *tiles_out = wdx::choose_tiles(N, (M + wdx::BM - 1) / wdx::BM, cus, K / kTileK / 4, grid);
  return hipSuccess;
}

hipError_t plan_gemm_linear(int M, int N, int K, size_t ws_bytes, int plan[4]) {
  plan[0] = 0;
  plan[1] = 0;
  plan[2] = 0;
  plan[3] = 1;
  if (!sk_shape(M, N, K)) return hipSuccess;
  int grid = 0, tiles = 0;
  const hipError_t err = wdx_plan(M, N, K, ws_bytes > 0, &grid, &tiles);
  if (err != hipSuccess) return err;
  const int rows = tiles == 3 ? wdx::kRows192 : tiles == 1 ? wdx::kRows128 : wdx::kRowsWide;
  const int T = (N / rows) * ((M + wdx::BM - 1) / wdx::BM);
  int R = 0, S = 1;
  wdx::split_plan(T, K / kTileK / 4, grid, &R, &S);
  plan[0] = rows;
  plan[1] = T;
  plan[2] = R;
  plan[3] = S;
  return hipSuccess;
}

hipError_t launch_gemm_linear(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                              Epilogue epi, const void* residual, int ldr, void* workspace, size_t ws_bytes,
                              hipStream_t stream) {
  if (sk_shape(M, N, K)) {
    // With a workspace, the partial last round is split over every CU (as
    // many as the workspace has partial slots for).
    int grid = 0, tiles = 0;
    const hipError_t err = wdx_plan(M, N, K, workspace != nullptr, &grid, &tiles);
    if (err != hipSuccess) return err;
    void* ws = grid > 0 ? workspace : nullptr;
    auto go = [&](auto a_tag, auto tb_tag) -> hipError_t {
      constexpr int A = decltype(a_tag)::value;
      constexpr int TB = decltype(tb_tag)::value;
      switch (epi) {
        case Epilogue::kSiluMul:
          return wdx::launch<1, A, TB>(w, N, K, x, M, ldx, y, ldy, residual, ldr, ws, grid, stream);
        case Epilogue::kResidualAdd:
          return wdx::launch<2, A, TB>(w, N, K, x, M, ldx, y, ldy, residual, ldr, ws, grid, stream);
        case Epilogue::kNone:
        default:
          return wdx::launch<0, A, TB>(w, N, K, x, M, ldx, y, ldy, residual, ldr, ws, grid, stream);
      }
    };
    // 256-row blocks run the (2, 8) wave tile: every wave over all 256
    // tokens, so each weight fragment is fetched by one wave only (4-9 %
    // faster than (4, 4), whose wave pairs fetched every weight line twice).
    if (tiles == 3) return go(std::integral_constant<int, 3>{}, std::integral_constant<int, 4>{});
    if (tiles == 1) return go(std::integral_constant<int, 1>{}, std::integral_constant<int, 8>{});
    return go(std::integral_constant<int, 2>{}, std::integral_constant<int, 8>{});
  }
  if (M > kGemmBM && N % big::BN == 0 && K % big::BK == 0) {
    switch (epi) {
      case Epilogue::kSiluMul:
        return big::launch<1>(w, N, K, x, M, ldx, y, ldy, residual, ldr, stream);
      case Epilogue::kResidualAdd:
        return big::launch<2>(w, N, K, x, M, ldx, y, ldy, residual, ldr, stream);
      case Epilogue::kNone:
      default:
        return big::launch<0>(w, N, K, x, M, ldx, y, ldy, residual, ldr, stream);
    }
  }
  switch (epi) {
    case Epilogue::kSiluMul:
      return launch_cfg<1>(w, N, K, x, M, ldx, y, ldy, residual, ldr, stream);
    case Epilogue::kResidualAdd:
      return launch_cfg<2>(w, N, K, x, M, ldx, y, ldy, residual, ldr, stream);
    case Epilogue::kNone:
    default:
      return launch_cfg<0>(w, N, K, x, M, ldx, y, ldy, residual, ldr, stream);
  }
}

}  // namespace lsk
