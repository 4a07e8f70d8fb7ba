// Persistent decode-step kernel: a whole sequence of projections (e.g. the
// 36 layers x {QKV, o_proj, gate_up + SiLU*up, down} of a decode or verify
// step at M <= 16) in ONE launch.
//
// Why: each projection is only 21-100 MB, 3-14 us of HBM time, so separate
// launches pay the ramp-up/tail of every kernel (about 2 us of fixed cost per
// launch even for an ideal streaming kernel).  Here one workgroup per CU
// walks a global list of work items in projection order, and every wave
// keeps the next chunk of weight tiles in flight while it computes the
// current one -- including across projection boundaries, where the weights
// of the next projection stream in while the wave waits for the previous
// projection's output (its activations).  Weights never depend on
// activations, so the dependency wait overlaps HBM traffic.
//
// Work item: one row-block group of one projection (16 output rows, or a
// 16-row gate/up pair for SiLU*up) over the full K.  The 8 waves of the
// workgroup split K, accumulate with v_mfma_f32_16x16x32_bf16 exactly as the
// single-projection decode kernel does (decode.hip), reduce through LDS in
// wave order (bitwise reproducible) and wave 0 applies the epilogue.
//
// Dependencies: projection p may name an earlier projection d whose output
// it reads.  Before the first chunk of an item of p, wave 0 of the workgroup
// polls done[q] for every q <= d until all their items are finished; the
// other waves wait at a barrier with their weight loads still in flight.
// After the epilogue, wave 0 waits for its output stores to complete and
// increments done[p].  Activations, residuals and outputs are read and
// written with coherent (agent-scope) accesses, so no cache maintenance is
// needed between producer and consumer workgroups.  The grid is sized to what the device holds at once
// (CUs x resident workgroups per CU, from the occupancy query), each
// workgroup processes its items in increasing projection order, so the
// dependency graph always drains; every wait is still bounded and records
// an error instead of spinning forever.  The last workgroup to
// finish resets the counters, so the workspace is reusable by the next
// launch (and by graph replays) without a memset.

#include <hip/hip_runtime.h>

#include "lsk_internal.h"

namespace lsk {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = kStackWaves;
constexpr int kChunkTiles = 12;         // weight tiles per wave per chunk (register budget)
constexpr unsigned kSpinLimit = 1u << 20;  // about a second of polling

// Pointers come from the program in memory, so the compiler cannot infer
// their address space; spell it out so weight loads are global_* ops.  (A
// flat load also counts in lgkmcnt, and every barrier's lgkmcnt(0) wait
// would then drain the whole weight prefetch.)
typedef __attribute__((address_space(1))) bf16x8_t global_bf16x8;

__device__ __forceinline__ bf16x8_t load_weight_tile(const bf16x8_t* p) {
  return __builtin_nontemporal_load((const global_bf16x8*)(p));
}

__device__ __forceinline__ bf16x8_t masked(bf16x8_t v, unsigned keep) {
  u32x4_t u = __builtin_bit_cast(u32x4_t, v);
  u &= keep;
  return __builtin_bit_cast(bf16x8_t, u);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_round(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

__device__ __forceinline__ unsigned short bf16_bits(float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}

__device__ __forceinline__ float silu_mul_bf16(float g_acc, float u_acc) {
  const float g = bf16_round(g_acc);
  const float u = bf16_round(u_acc);
  const float s = bf16_round(g / (1.0f + expf(-g)));
  return bf16_round(s * u);
}

// Wave-uniform position in the chunk sequence.
struct Cursor {
  int gi;     // global item index (>= total: finished)
  int p;      // projection of the item
  int item;   // item index inside projection p
  int kb;     // first k-tile of this wave's range of the item
  int len;    // k-tiles in this wave's range
  int nc;     // chunks the range is cut into (balanced sizes)
  int ci;     // current chunk
  int kt0;    // first k-tile of the chunk
  int nkt;    // k-tiles in the chunk
  int first;  // 1 on the first chunk of this wave's part of the item
};

struct Ctx {
  const StackDesc* desc;
  int count;
  int total;
  int wave;
  int lane;
};

__device__ __forceinline__ void set_chunk(Cursor& c) {
  c.kt0 = c.kb + (c.len * c.ci) / c.nc;
  c.nkt = c.kb + (c.len * (c.ci + 1)) / c.nc - c.kt0;
}

// Start the wave's part of global item gi (searching forward from projection p).
// Every wave's range has the same length (K/32 is a multiple of the wave
// count), so all waves see the same chunk count and meet at the same barriers.
__device__ __forceinline__ void open_item(Cursor& c, const Ctx& x, int gi, int p) {
  c.gi = gi;
  if (gi >= x.total) return;
  while (p + 1 < x.count && gi >= x.desc[p + 1].item_begin) ++p;
  c.p = p;
  c.item = gi - x.desc[p].item_begin;
  c.len = x.desc[p].KT / kWaves;
  c.kb = c.len * x.wave;
  const int cap = kChunkTiles / x.desc[p].rbw;
  c.nc = (c.len + cap - 1) / cap;
  c.ci = 0;
  c.first = 1;
  set_chunk(c);
}

__device__ __forceinline__ void advance(Cursor& c, const Ctx& x) {
  if (c.ci + 1 < c.nc) {
    ++c.ci;
    c.first = 0;
    set_chunk(c);
  } else {
    open_item(c, x, c.gi + gridDim.x, c.p);
  }
}

__device__ __forceinline__ bool is_last(const Cursor& c) { return c.ci + 1 == c.nc; }

__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
  return (unsigned)bf16_bits(lo) | ((unsigned)bf16_bits(hi) << 16);
}

template <int RBW>
__device__ __forceinline__ void issue_weights(bf16x8_t (&buf)[kChunkTiles], const StackDesc& d, const Cursor& c,
                                              int lane) {
  const bf16x8_t* base = d.w + ((size_t)c.item * RBW * d.KT + c.kt0) * 64 + lane;
#pragma unroll
  for (int t = 0; t < kChunkTiles / RBW; ++t) {
    if (t < c.nkt) {
#pragma unroll
      for (int r = 0; r < RBW; ++r) buf[t * RBW + r] = load_weight_tile(base + ((size_t)r * d.KT + t) * 64);
    }
  }
}

// Activations and outputs cross workgroups (and XCDs, whose L2s are not
// coherent with each other), so every access to them is an agent-scope
// relaxed atomic: coherent loads and stores that need no L2 write-back or
// invalidate.  (Fence-based release/acquire would write back and invalidate
// a whole L2 per item, which costs far more than the item itself.)
// Global-address-space view, so these become global_* (not flat_*) ops.
typedef __attribute__((address_space(1))) unsigned long long global_u64;

__device__ __forceinline__ unsigned long long coherent_load64(const void* p) {
  return __hip_atomic_load((const global_u64*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void coherent_store64(void* p, unsigned long long v) {
  __hip_atomic_store((global_u64*)(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bf16x8_t coherent_frag(const bf16x8_t* p, unsigned long long keep) {
  const unsigned long long lo = coherent_load64(p) & keep;
  const unsigned long long hi = coherent_load64(reinterpret_cast<const unsigned long long*>(p) + 1) & keep;
  u32x4_t u{(unsigned)lo, (unsigned)(lo >> 32), (unsigned)hi, (unsigned)(hi >> 32)};
  return __builtin_bit_cast(bf16x8_t, u);
}

__device__ __forceinline__ void issue_x(bf16x8_t (&xv)[kChunkTiles], const StackDesc& d, const Cursor& c, int M,
                                        int lane) {
  const int m = lane & 15;
  const int g = lane >> 4;
  const unsigned long long keep = m < M ? ~0ull : 0ull;
  const bf16x8_t* row = reinterpret_cast<const bf16x8_t*>(d.x + (size_t)(m < M ? m : 0) * d.ldx) + g;
  const int cap = kChunkTiles / d.rbw;
#pragma unroll
  for (int t = 0; t < kChunkTiles; ++t) {
    if (t < c.nkt && t < cap) xv[t] = coherent_frag(row + (c.kt0 + t) * 4, keep);
  }
}

template <int RBW>
__device__ __forceinline__ void consume(f32x4_t (&acc)[2], const bf16x8_t (&buf)[kChunkTiles],
                                        const bf16x8_t (&xv)[kChunkTiles], int nkt) {
#pragma unroll
  for (int t = 0; t < kChunkTiles / RBW; ++t) {
    if (t < nkt) {
#pragma unroll
      for (int r = 0; r < RBW; ++r) acc[r] = mfma16(buf[t * RBW + r], xv[t], acc[r]);
    }
  }
}

// Wave 0, after the LDS reduction: write the item's outputs and publish it.
__device__ __forceinline__ void finish_item(const StackDesc& d, int item, const f32x4_t (&acc)[2], int M, int lane,
                                            unsigned* done_p) {
  const int m = lane & 15;
  const int g = lane >> 4;
  if (m < M) {
    const int n = item * 16 + 4 * g;  // output column (intermediate index for SiLU*up)
    f32x4_t v;
    if (d.epi == static_cast<int>(Epilogue::kSiluMul)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = silu_mul_bf16(acc[0][i], acc[1][i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = bf16_round(acc[0][i]);
      if (d.epi == static_cast<int>(Epilogue::kResidualAdd)) {
        const unsigned long long r = coherent_load64(d.res + (size_t)m * d.ldr + n);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[i] += __builtin_bit_cast(float, (unsigned)((r >> (16 * i)) & 0xffffu) << 16);
      }
    }
    const unsigned long long packed =
        (unsigned long long)pack_bf16x2(v[0], v[1]) | ((unsigned long long)pack_bf16x2(v[2], v[3]) << 32);
    coherent_store64(d.y + (size_t)m * d.ldy + n, packed);
  }
  // Publish: the wave's output stores have completed (vmcnt counts stores on
  // this target) before the item counter moves.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (lane == 0) __hip_atomic_fetch_add(done_p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0: wait until projection `dep` has published all of its items.
// Once any wait of the launch has given up, later waits return at once, so a
// broken program ends in about one spin limit rather than one per projection.
__device__ __forceinline__ void wait_projection(unsigned* done_dep, unsigned target, unsigned* error) {
  unsigned spins = 0;
  while (__hip_atomic_load(done_dep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
    if (__hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
    __builtin_amdgcn_s_sleep(2);
    if (++spins > kSpinLimit) {
      __hip_atomic_store(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
  }
  asm volatile("" ::: "memory");  // keep the activation loads after the wait
}

__global__ __launch_bounds__(kWaves * 64, 1) void decode_stack_kernel(const StackProgram* __restrict__ prog,
                                                                       unsigned* __restrict__ ws) {
  // Cross-wave reduction slots (dynamic LDS, two alternating item slots).
  extern __shared__ f32x4_t lds_dyn[];
  f32x4_t (*red)[kWaves - 1][2][64] = reinterpret_cast<f32x4_t (*)[kWaves - 1][2][64]>(lds_dyn);
  __shared__ int s_dep_ok;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int M = prog->M;
  if (prog->magic != kStackMagic) {
    if (threadIdx.x == 0) __hip_atomic_store(ws + kStackWsError, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  unsigned* done = ws + kStackWsCounters;
  unsigned* error = ws + kStackWsError;
  unsigned* exit_count = ws + kStackWsExit;

  Ctx x{prog->desc, prog->count, prog->total_items, wave, lane};
  if (threadIdx.x == 0) s_dep_ok = -1;  // highest projection whose input wait is done

  Cursor cur;
  open_item(cur, x, blockIdx.x, 0);
  bf16x8_t buf0[kChunkTiles], buf1[kChunkTiles], xv[kChunkTiles];
  f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
  int red_slot = 0;
  __syncthreads();

  if (cur.gi < x.total) {
    const StackDesc& d = x.desc[cur.p];
    if (d.rbw == 1) issue_weights<1>(buf0, d, cur, lane); else issue_weights<2>(buf0, d, cur, lane);
  }

  // One pipeline step: compute chunk `cur` (weights in `mine`), having first
  // issued the next chunk's weights into `other`.
  auto step = [&](bf16x8_t (&mine)[kChunkTiles], bf16x8_t (&other)[kChunkTiles]) {
    const StackDesc& d = x.desc[cur.p];
    if (cur.first && d.dep > s_dep_ok) {
      // Input comes from earlier projections: wave 0 acquires every
      // projection up to d.dep, the other waves wait here with their weight
      // loads in flight.
      if (wave == 0) {
        for (int q = s_dep_ok + 1; q <= d.dep; ++q) wait_projection(done + q, (unsigned)x.desc[q].items, error);
        if (lane == 0) s_dep_ok = d.dep;
      }
      __syncthreads();
    }
    issue_x(xv, d, cur, M, lane);
    Cursor nxt = cur;
    advance(nxt, x);
    if (nxt.gi < x.total) {
      const StackDesc& dn = x.desc[nxt.p];
      if (dn.rbw == 1) issue_weights<1>(other, dn, nxt, lane); else issue_weights<2>(other, dn, nxt, lane);
    }
    if (d.rbw == 1) consume<1>(acc, mine, xv, cur.nkt); else consume<2>(acc, mine, xv, cur.nkt);
    if (is_last(cur)) {
      // Reduce the item's 8 partial tiles in wave order (LDS slot alternates
      // so wave 0 can still be reading the previous item's slot).
      if (wave > 0) {
        red[red_slot][wave - 1][0][lane] = acc[0];
        red[red_slot][wave - 1][1][lane] = acc[1];
      }
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int w = 0; w < kWaves - 1; ++w) {
          acc[0] += red[red_slot][w][0][lane];
          acc[1] += red[red_slot][w][1][lane];
        }
        finish_item(d, cur.item, acc, M, lane, done + cur.p);
      }
      red_slot ^= 1;
      acc[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      acc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    cur = nxt;
  };

  while (cur.gi < x.total) {
    step(buf0, buf1);
    if (cur.gi >= x.total) break;
    step(buf1, buf0);
  }

  // Last workgroup out resets the counters for the next launch.
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(exit_count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gridDim.x - 1) {
      for (int p = 0; p < x.count; ++p) __hip_atomic_store(done + p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(exit_count, 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

size_t stack_lds_bytes() { return sizeof(f32x4_t) * 2 * (kWaves - 1) * 2 * 64; }

const void* stack_kernel_symbol() { return reinterpret_cast<const void*>(&decode_stack_kernel); }

hipError_t launch_decode_stack(const StackProgram* prog, unsigned* ws, int grid, size_t lds_bytes,
                               hipStream_t stream) {
  decode_stack_kernel<<<dim3(grid), dim3(kWaves * 64), lds_bytes, stream>>>(prog, ws);
  return hipGetLastError();
}

}  // namespace lsk
