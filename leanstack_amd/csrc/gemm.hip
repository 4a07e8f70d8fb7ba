// Prefill projections (M in the hundreds to thousands) on gfx950 MFMA.
//
// y[M][N] = epilogue(x[M][K] . W[N][K]^T) with W in LSK_LAYOUT_MFMA16X32.
// Because each packed 1 KB weight tile already is a v_mfma_f32_16x16x32_bf16
// operand in lane order, the weight half of every LDS stage is a straight
// linear copy (no swizzle, no bank conflicts on write or read).  The
// activation half is re-tiled into the same 16x32 operand order as it is
// copied into LDS, so both MFMA operands are read with linear 16-byte LDS
// loads.
//
// Block tile 128 (weight rows) x 128 (tokens) x 64 (K), 4 wavefronts in a 2x2
// arrangement, each owning 64x64 = 4x4 MFMA tiles; LDS is double buffered so
// the global loads of stage s+1 are in flight while stage s is multiplied.
// Workgroups are remapped so that each XCD walks a contiguous run of the
// (weight block, token block) space: the token blocks sharing one weight
// block then share that XCD's L2.
//
// Reference arithmetic replaced: F.linear at
// src/leanstack/runtime/qwen_explicit.py:748, :819, :828, :830, :1202-1208 and
// the cuTile GEMM of experiments/cutile/qwen_bf16_hot_kernels.py:24-36.

#include <hip/hip_runtime.h>

#include "lsk_internal.h"

namespace lsk {
namespace {

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

__device__ __forceinline__ bf16x8_t zero_frag() {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_round(float v) {
  return static_cast<float>(static_cast<__bf16>(v));
}

__device__ __forceinline__ unsigned short bf16_bits(float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}

__device__ __forceinline__ float silu_mul_bf16(float g_acc, float u_acc) {
  const float g = bf16_round(g_acc);
  const float u = bf16_round(u_acc);
  const float s = bf16_round(g / (1.0f + expf(-g)));
  return bf16_round(s * u);
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
    r.v[4 + j] = row < M ? *reinterpret_cast<const bf16x8_t*>(x + (size_t)row * ldx + k) : zero_frag();
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

  // XCD-aware remap: workgroup b runs on XCD b % 8; give each XCD a
  // contiguous run of logical tiles (weight-block major).
  const int total = n_blocks * m_blocks;
  int logical = blockIdx.x;
  if (total % 8 == 0) logical = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
  const int nb = logical / m_blocks;
  const int mb = logical % m_blocks;

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

  for (int s = 0; s < stages; ++s) {
    const int cur = s & 1;
    const bool more = s + 1 < stages;
    if (more) load_stage(regs, w, x, ldx, M, KT, rb_base, m_base, (s + 1) * kKtPerStage, wave, lane);
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
    if (more) store_stage(lds[cur ^ 1], regs, wave, lane);
    __syncthreads();
  }

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

template <int EPI>
hipError_t launch_cfg(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                      const void* residual, int ldr, hipStream_t stream) {
  const int n_blocks = N / kGemmBN;
  const int m_blocks = (M + kGemmBM - 1) / kGemmBM;
  gemm_linear_kernel<EPI><<<dim3(n_blocks * m_blocks), dim3(kThreads), 0, stream>>>(
      static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, static_cast<__bf16*>(y), ldy,
      static_cast<const __bf16*>(residual), ldr, M, K / kTileK, n_blocks, m_blocks);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_linear(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                              Epilogue epi, const void* residual, int ldr, hipStream_t stream) {
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
