// Projections of 17..128 rows on gfx950: y[M][N] = epilogue(x[M][K] . W^T).
//
// At these row counts a projection is still bound by its weight bytes (the
// arithmetic intensity is M FLOP per weight byte, under 128), so the kernel
// keeps the decode kernels' streaming form and widens its B operand instead
// of tiling like the prefill GEMM: every packed 1 KB weight tile is loaded
// once, straight into registers as the A operand of
// v_mfma_f32_16x16x32_bf16, and multiplied with ceil(M / 16) activation
// fragments of 16 tokens each (MG groups), read from L2 next to it.
//
// Work split.  A workgroup owns RBW row-blocks (16 output rows each; a
// gate/up pair for SiLU*up) over one K range; its 8 wavefronts split that
// range and their partial tiles are summed through LDS in wave order.  When
// the row-blocks alone would leave CUs idle (kv/o/down-sized N), the call's
// workspace lets the K range of every row-block be split over S workgroups:
// each publishes its fp32 partial with device-coherent stores and counts its
// arrival, and the workgroup that arrives last adds the S partials in split
// order, applies the epilogue and stores the rows.  Nothing waits on another
// workgroup, and every sum has a fixed order, so results are bitwise
// reproducible; the split form and the unsplit one add in different orders
// and agree to fp32 rounding.
//
// Reference arithmetic replaced: F.linear at
// src/leanstack/runtime/qwen_explicit.py:748, :819, :828-830, :1202-1208 for
// the verify and short prefill batches, and the hot-kernel GEMM cases of
// src/leanstack/hot_kernels.py:81-194 (M = 64).

#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>
#include <vector>

#include "lsk_internal.h"

namespace lsk {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kNW = kSkinnyWaves;  // wavefronts per workgroup
constexpr int kCoherent = 16;      // buffer cache policy: device-coherent (sc1)

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// k-tiles loaded per round: about 16 loads per wave in flight.
template <int RBW, int MG>
constexpr int round_tiles() {
  return 16 / (RBW + MG) > 0 ? 16 / (RBW + MG) : 1;
}

// Token groups summed per LDS round: the largest divisor of MG with
// RBW * CG <= 8 (7 waves x 8 KB of partial tiles).
template <int RBW, int MG>
constexpr int sum_chunk() {
  int c = 8 / RBW < MG ? 8 / RBW : MG;
  while (MG % c != 0) --c;
  return c;
}

template <int RBW, int MG, int EPI>
__global__ __launch_bounds__(kNW * 64) void skinny_kernel(
    const bf16x8_t* __restrict__ w, const __bf16* __restrict__ x, int ldx, __bf16* __restrict__ y, int ldy,
    const __bf16* __restrict__ residual, int ldr, int M, int KT, int S, unsigned* __restrict__ counters,
    unsigned char* __restrict__ partials, unsigned partial_bytes) {
  static_assert(EPI != static_cast<int>(Epilogue::kSiluMul) || RBW % 2 == 0,
                "SiLU*up takes whole gate/up pairs of row-blocks");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m = lane & 15;  // B-operand column = token within its group
  const int g = lane >> 4;  // K group inside a tile / output row quad
  const int grp = blockIdx.x / S;
  const int split = blockIdx.x - grp * S;
  const int rb0 = grp * RBW;
  const int sb = (KT * split) / S, se = (KT * (split + 1)) / S;
  const int kb = sb + ((se - sb) * wave) / kNW;
  const int ke = sb + ((se - sb) * (wave + 1)) / kNW;

  f32x4_t acc[RBW][MG];
#pragma unroll
  for (int r = 0; r < RBW; ++r)
#pragma unroll
    for (int q = 0; q < MG; ++q) acc[r][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Token rows 16q + m; rows past M read row 0 (in bounds) and are masked.
  const bf16x8_t* xr[MG];
  unsigned keep[MG];
#pragma unroll
  for (int q = 0; q < MG; ++q) {
    const int row = 16 * q + m;
    keep[q] = row < M ? 0xffffffffu : 0u;
    xr[q] = reinterpret_cast<const bf16x8_t*>(x + (size_t)(row < M ? row : 0) * ldx) + g;
  }
  const bf16x8_t* wt = w + (size_t)rb0 * KT * 64 + lane;

  // Rounds of R k-tiles: every load of a round goes out before its first
  // multiply, so each wave keeps about 16 loads in flight.
  constexpr int R = round_tiles<RBW, MG>();
  auto round = [&](int kt, auto n_tag) {
    constexpr int N = decltype(n_tag)::value;
    bf16x8_t wv[N][RBW];
    bf16x8_t xv[N][MG];
#pragma unroll
    for (int u = 0; u < N; ++u)
#pragma unroll
      for (int r = 0; r < RBW; ++r) wv[u][r] = __builtin_nontemporal_load(wt + ((size_t)r * KT + kt + u) * 64);
#pragma unroll
    for (int u = 0; u < N; ++u)
#pragma unroll
      for (int q = 0; q < MG; ++q) {
        u32x4_t v = __builtin_bit_cast(u32x4_t, xr[q][(kt + u) * 4]);
        v &= keep[q];
        xv[u][q] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
    for (int u = 0; u < N; ++u)
#pragma unroll
      for (int r = 0; r < RBW; ++r)
#pragma unroll
        for (int q = 0; q < MG; ++q) acc[r][q] = mfma16(wv[u][r], xv[u][q], acc[r][q]);
  };
  int kt = kb;
  for (; kt + R <= ke; kt += R) round(kt, std::integral_constant<int, R>{});
  for (; kt < ke; ++kt) round(kt, std::integral_constant<int, 1>{});

  // Cross-wave sum in wave order, CG token groups at a time (56 KB of LDS).
  constexpr int CG = sum_chunk<RBW, MG>();
  static_assert(MG % CG == 0, "token groups are summed in whole chunks");
  __shared__ f32x4_t red[kNW - 1][RBW * CG][64];
#pragma unroll
  for (int c0 = 0; c0 < MG; c0 += CG) {
    if (wave > 0) {
#pragma unroll
      for (int r = 0; r < RBW; ++r)
#pragma unroll
        for (int j = 0; j < CG; ++j) red[wave - 1][r * CG + j][lane] = acc[r][c0 + j];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int v = 0; v < kNW - 1; ++v)
#pragma unroll
        for (int r = 0; r < RBW; ++r)
#pragma unroll
          for (int j = 0; j < CG; ++j) acc[r][c0 + j] += red[v][r * CG + j][lane];
    }
    if (c0 + CG < MG) __syncthreads();
  }
  if (wave != 0) return;

  if (S > 1) {
    // Publish this split's partial, count the arrival; the last of the S
    // splits of the row-blocks sums them in split order.  Partials cross
    // XCDs, whose L2s are not coherent with each other: device-coherent
    // buffer stores and loads, and the arrival only after the stores are
    // acknowledged.
    const __amdgpu_buffer_rsrc_t parts =
        __builtin_amdgcn_make_buffer_rsrc(partials, (short)0, (int)partial_bytes, (int)0x00020000u);
    constexpr unsigned kSlot = RBW * MG * 64 * 16;
#pragma unroll
    for (int r = 0; r < RBW; ++r)
#pragma unroll
      for (int q = 0; q < MG; ++q)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[r][q]), parts, lane * 16,
                                               (unsigned)blockIdx.x * kSlot + (r * MG + q) * 1024u, kCoherent);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(counters + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
    if (old != (unsigned)S - 1) return;
    // Last arrival: every other split's partial is acknowledged.  Re-arm the
    // counter for the next call, then add the S partials in split order, this
    // split's own from its registers.  The others are loaded PB partials at a
    // time (16 fragments in flight); slots past the last split are read at an
    // offset beyond the buffer's range, which returns zeros without a memory
    // access, and are never added.
    if (lane == 0) __hip_atomic_store(counters + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    constexpr int PB = RBW * MG >= 16 ? 1 : 16 / (RBW * MG);
    f32x4_t mine[RBW][MG];
#pragma unroll
    for (int r = 0; r < RBW; ++r)
#pragma unroll
      for (int q = 0; q < MG; ++q) {
        mine[r][q] = acc[r][q];
        acc[r][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    bool own_added = false;
    for (int o0 = 0; o0 < S - 1; o0 += PB) {
      f32x4_t v[PB][RBW][MG];
#pragma unroll
      for (int b = 0; b < PB; ++b) {
        const int o = o0 + b;  // o-th other split in split order
        const int sp = o < split ? o : o + 1;
        // Out of range goes in the vector offset: the range check covers the
        // vector and instruction offsets, not the scalar one.
        const bool real = o < S - 1;
        const unsigned voff = (real ? 0u : 0x80000000u) + (unsigned)lane * 16u;
        const unsigned base = real ? (unsigned)(grp * S + sp) * kSlot : 0u;
#pragma unroll
        for (int r = 0; r < RBW; ++r)
#pragma unroll
          for (int q = 0; q < MG; ++q)
            v[b][r][q] = __builtin_bit_cast(
                f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(parts, voff, base + (r * MG + q) * 1024u, kCoherent));
      }
#pragma unroll
      for (int b = 0; b < PB; ++b) {
        const int o = o0 + b;
        if (o >= S - 1) break;
        if (!own_added && (o < split ? o : o + 1) > split) {
#pragma unroll
          for (int r = 0; r < RBW; ++r)
#pragma unroll
            for (int q = 0; q < MG; ++q) acc[r][q] += mine[r][q];
          own_added = true;
        }
#pragma unroll
        for (int r = 0; r < RBW; ++r)
#pragma unroll
          for (int q = 0; q < MG; ++q) acc[r][q] += v[b][r][q];
      }
    }
    if (!own_added) {
#pragma unroll
      for (int r = 0; r < RBW; ++r)
#pragma unroll
        for (int q = 0; q < MG; ++q) acc[r][q] += mine[r][q];
    }
  }

  // Lane (g, m) holds output rows 4g..4g+3 of each row-block for token
  // 16q + m of each group q.
#pragma unroll
  for (int q = 0; q < MG; ++q) {
    const int tok = 16 * q + m;
    if (tok >= M) continue;
    if constexpr (EPI == static_cast<int>(Epilogue::kSiluMul)) {
#pragma unroll
      for (int p = 0; p < RBW / 2; ++p) {
        const int j = (rb0 / 2 + p) * 16 + 4 * g;  // intermediate index
        unsigned short o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = bf16_bits(silu_mul_bf16(acc[2 * p][q][i], acc[2 * p + 1][q][i]));
        *reinterpret_cast<u32x2_t*>(y + (size_t)tok * ldy + j) =
            u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
      }
    } else {
#pragma unroll
      for (int r = 0; r < RBW; ++r) {
        const int n = (rb0 + r) * 16 + 4 * g;
        unsigned short o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = bf16_round(acc[r][q][i]);
          if constexpr (EPI == static_cast<int>(Epilogue::kResidualAdd))
            v = static_cast<float>(residual[(size_t)tok * ldr + n + i]) + v;
          o[i] = bf16_bits(v);
        }
        *reinterpret_cast<u32x2_t*>(y + (size_t)tok * ldy + n) =
            u32x2_t{o[0] | ((unsigned)o[1] << 16), o[2] | ((unsigned)o[3] << 16)};
      }
    }
  }
}

template <int RBW, int MG, int EPI>
hipError_t launch_cfg(const SkinnyPlan& p, const void* w, const void* x, int ldx, void* y, int ldy,
                      const void* residual, int ldr, int M, int KT, void* workspace, hipStream_t stream) {
  auto* ws = static_cast<unsigned char*>(workspace);
  unsigned* counters = p.S > 1 ? reinterpret_cast<unsigned*>(ws + kSkFlagsOffset) : nullptr;
  unsigned char* partials = p.S > 1 ? ws + kSkPartialsOffset : nullptr;
  const unsigned partial_bytes = p.S > 1 ? (unsigned)(p.groups * p.S * RBW * MG * 1024) : 0u;
  launch_kernel(skinny_kernel<RBW, MG, EPI>, dim3(p.groups * p.S), dim3(kNW * 64), 0, stream,
                static_cast<const bf16x8_t*>(w), static_cast<const __bf16*>(x), ldx, static_cast<__bf16*>(y), ldy,
                static_cast<const __bf16*>(residual), ldr, M, KT, p.S, counters, partials, partial_bytes);
  return hipGetLastError();
}

template <int RBW, int EPI>
hipError_t launch_rbw(const SkinnyPlan& p, const void* w, const void* x, int ldx, void* y, int ldy,
                      const void* residual, int ldr, int M, int KT, void* workspace, hipStream_t stream) {
  switch (skinny_groups(M)) {
    case 2:
      return launch_cfg<RBW, 2, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
    case 3:
      return launch_cfg<RBW, 3, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
    case 4:
      return launch_cfg<RBW, 4, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
    case 6:
      if constexpr (RBW <= 2) return launch_cfg<RBW, 6, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
      break;
    case 8:
      if constexpr (RBW <= 2) return launch_cfg<RBW, 8, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
      break;
    default:
      break;
  }
  return hipErrorInvalidValue;
}

template <int EPI>
hipError_t launch_epi(const SkinnyPlan& p, const void* w, const void* x, int ldx, void* y, int ldy,
                      const void* residual, int ldr, int M, int KT, void* workspace, hipStream_t stream) {
  const int rbw = p.rows / kTileRows;
  if (rbw == 4) return launch_rbw<4, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
  if (rbw == 2) return launch_rbw<2, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
  if constexpr (EPI != static_cast<int>(Epilogue::kSiluMul))
    return launch_rbw<1, EPI>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
  return hipErrorInvalidValue;
}

}  // namespace

// CUs of the current device (cached per device): the skinny split covers them.
hipError_t current_device_cus(int* cus_out) {
  static std::mutex mu;
  static std::vector<int> cache;
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return err;
  std::lock_guard<std::mutex> lock(mu);
  if (device >= (int)cache.size()) cache.resize(device + 1, 0);
  if (cache[device] == 0) {
    int cus = 0;
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (err != hipSuccess) return err;
    cache[device] = cus > 0 ? cus : 1;
  }
  *cus_out = cache[device];
  return hipSuccess;
}

// Token groups a call of M rows computes (5 and 7 run as 6 and 8: the LDS
// sum takes whole chunks).
int skinny_groups(int M) {
  const int mg = (M + kTileRows - 1) / kTileRows;
  return mg == 5 ? 6 : mg == 7 ? 8 : mg;
}

// Whether lsk_linear_bf16 runs M rows of an [N, K] projection on the skinny
// kernel: 17..64 rows always, 65..128 rows unless N is wide enough (>= 8192,
// the gate_up shapes) for the 128 x 128 GEMM's blocks to fill the chip, which
// then reads each activation fragment once per 128 weight rows instead of
// once per 32 (measured at 128 rows: gate_up 9728 x 2560 38 against 58 us,
// the fused 19456 x 2560 with SiLU*up 40 against 92 us).
bool skinny_route(int M, int N, int K) {
  if (M <= kDecodeMaxM || M > kSkinnyMaxM || N % kTileRows != 0 || K % kTileK != 0) return false;
  const bool gemm_grid = N % kGemmBN == 0 && K % kGemmBK == 0;
  return M <= 64 || !gemm_grid || N < 8192;
}

// Row-blocks per workgroup and the K split, from a sweep of every (rows, S)
// over the Qwen3-4B projections at 17, 32, 64 and 128 rows on 256 CUs: two
// row-blocks (one gate/up pair) per workgroup by default, since each
// activation fragment is read once for all of them; one for narrow N (fewer
// than 64 pairs of row-blocks) and for up to 32 rows when the row-blocks
// alone cover every CU; four (up to 64 rows, for the registers) when two
// would take more than one round of the CUs and four still cover half of
// them.  With a workspace the K range is split so that the grid comes to
// about one workgroup per CU, each split keeping at least two k-tiles per
// wave.
SkinnyPlan skinny_plan(int M, int N, int K, bool silu, int cus, bool has_workspace) {
  const int NB = N / kTileRows;
  const int KT = K / kTileK;
  const int mg = skinny_groups(M);
  int rbw = 2;
  if (!silu && ((mg <= 2 && NB >= cus) || NB / 2 < 64 || NB % 2 != 0)) {
    rbw = 1;
  } else if (mg <= 4 && NB % 4 == 0 && NB / 2 > cus && NB / 4 <= cus && 2 * (NB / 4) >= cus) {
    rbw = 4;
  }
  const int groups = NB / rbw;
  int S = 1;
  const int max_s = KT / (2 * kNW);
  if (has_workspace && groups <= kSkinnyMaxGroups && max_s >= 2) {
    S = (4 * cus + groups) / (4 * groups);  // floor(cus / groups + 1/4)
    if (S > max_s) S = max_s;
    if (S < 1) S = 1;
  }
  SkinnyPlan p;
  p.rows = kTileRows * rbw;
  p.groups = NB / rbw;
  p.S = S;
  p.bytes = p.S > 1 ? kSkPartialsOffset + (size_t)p.groups * p.S * rbw * mg * 1024 : 0;
  return p;
}

hipError_t launch_skinny_linear(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                                Epilogue epi, const void* residual, int ldr, void* workspace, size_t ws_bytes,
                                int cus, hipStream_t stream) {
  const bool silu = epi == Epilogue::kSiluMul;
  SkinnyPlan p = skinny_plan(M, N, K, silu, cus, workspace != nullptr);
  if (p.S > 1 && ws_bytes < p.bytes) return hipErrorInvalidValue;  // checked by the caller
  const int KT = K / kTileK;
  switch (epi) {
    case Epilogue::kSiluMul:
      return launch_epi<1>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
    case Epilogue::kResidualAdd:
      return launch_epi<2>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
    case Epilogue::kNone:
    default:
      return launch_epi<0>(p, w, x, ldx, y, ldy, residual, ldr, M, KT, workspace, stream);
  }
}

}  // namespace lsk
