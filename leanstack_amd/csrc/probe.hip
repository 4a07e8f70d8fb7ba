// Measurement kernels: lsk_probe_stream_step (the decode step's launch
// structure, bench.py --probe-step-floor) and lsk_probe_mfma_rate (the dense
// BF16 MFMA rate with no memory traffic, bench.py --probe-mfma).  No
// counterpart in the reference.
//
// It answers one question about a single-launch (persistent) decode step:
// how fast can one workgroup per CU stream a step's weight bytes when every
// projection must wait for the whole previous one?  Segment s stands for
// projection s: each CU streams its equal share of the segment's 1 KB tiles
// through W compute waves (a ring of R tiles in flight per wave, each tile
// multiplied into an accumulator so the loads are consumed as the decode
// kernels consume them).  A control wave per workgroup runs the dependency:
//   mode 0  none (the streaming rate of this structure);
//   mode 1  a flat barrier: every workgroup counts its arrival on one word
//           per segment and polls it until all have arrived;
//   mode 2  a two-level barrier: arrivals on 8 group words, the last arrival
//           of each group counts on one global word, polls it and releases
//           its group through a go word that the group polls;
//   mode 3  tag words: every workgroup stores segment + 1 into its own word
//           of 8 replicas of a tag array and polls the whole array of its
//           replica (workgroup & 7) until every word has reached it: one
//           store and one load round trip per boundary, no atomics.
// Compute waves wait (in LDS) for the control wave before multiplying the
// first tile of a segment, but their ring of weight loads runs ahead across
// the wait.  Nothing is stored but a checksum; every wait is bounded.

#include <hip/hip_runtime.h>

#include "lsk_internal.h"

namespace lsk {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) unsigned global_u32;

constexpr int kW = kProbeComputeWaves;
constexpr unsigned kSpin = 1u << 20;

template <int I>
struct IntC {
  static constexpr int value = I;
};
template <int N, int I = 0, typename F>
__device__ __forceinline__ void unroll(F&& f) {
  if constexpr (I < N) {
    f(IntC<I>{});
    unroll<N, I + 1>(f);
  }
}

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load((const global_u32*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned* p, unsigned v) {
  __hip_atomic_store((global_u32*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_agent(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add((global_u32*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned lds_load(unsigned* p) {
  return (unsigned)__builtin_amdgcn_readfirstlane((int)__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}
__device__ __forceinline__ void lds_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The least of words t[0..n) (n <= 256, agent scope, 4 per lane), uniform.
__device__ __forceinline__ unsigned min_words(const unsigned* t, int n, int lane) {
  unsigned m = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (lane + 64 * i < n) m = min(m, ld_agent(t + lane + 64 * i));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = min(m, (unsigned)__shfl_xor((int)m, o));
  return (unsigned)__builtin_amdgcn_readfirstlane((int)m);
}

// Waits until *p >= target (agent scope), or gives up: the error word is set
// and every later wait of the launch returns at once.
__device__ __forceinline__ void wait_at_least(const unsigned* p, unsigned target, unsigned* error) {
  unsigned spins = 0;
  while (ld_agent(p) < target) {
    if (ld_agent(error) != 0u) return;
    __builtin_amdgcn_s_sleep(1);
    if (++spins > kSpin) {
      st_agent(error, 1u);
      return;
    }
  }
}

template <int R, int MODE>
__global__ __launch_bounds__((kW + 1) * 64, 1) void probe_step_kernel(const char* __restrict__ wbase, ProbeSegments seg,
                                                                       unsigned* __restrict__ ws) {
  __shared__ unsigned done[kW], ready;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = blockIdx.x, G = gridDim.x;
  const int S = seg.count;
  if (threadIdx.x < kW) done[threadIdx.x] = 0;
  if (threadIdx.x == 0) ready = 0;
  __syncthreads();
  unsigned* error = ws + kProbeWsError;
  if (wave < kW) {
    // Tile j = wave, wave + W, ... of this CU's share of every segment.
    struct Cursor {
      int s, j;
      size_t tile;
    };
    auto seg_tile = [&](int s, int j) -> size_t { return seg.first[s] + (size_t)c * seg.per_cu[s] + j; };
    Cursor ld{0, wave, seg_tile(0, wave)};
    auto advance = [&](Cursor& q) {
      q.j += kW;
      q.tile += kW;
      if (q.j >= seg.per_cu[q.s]) {
        ++q.s;
        q.j = wave;
        q.tile = q.s < S ? seg_tile(q.s, wave) : 0;  // past the end: tile 0, never multiplied
      }
    };
    const char* lbase = wbase + lane * 16;
    bf16x8_t ring[R];
    unroll<R>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      ring[k] = __builtin_bit_cast(bf16x8_t, __builtin_nontemporal_load((const u32x4_t*)(lbase + ld.tile * 1024)));
      advance(ld);
    });
    int cs = 0, cj = wave;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    const bf16x8_t xf = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    while (cs < S) {
      unroll<R>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if (cs < S) {
          if (MODE > 0 && cj == wave && cs > 0) {
            unsigned spins = 0;
            while (lds_load(&ready) < (unsigned)cs) {
              __builtin_amdgcn_s_sleep(1);
              if (++spins > 4 * kSpin) break;
            }
          }
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ring[k], xf, acc, 0, 0, 0);
          cj += kW;
          if (cj >= seg.per_cu[cs]) {
            lds_store(&done[wave], (unsigned)cs + 1);
            ++cs;
            cj = wave;
          }
        }
        ring[k] = __builtin_bit_cast(bf16x8_t, __builtin_nontemporal_load((const u32x4_t*)(lbase + ld.tile * 1024)));
        advance(ld);
      });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // A checksum nobody expects to match, so the multiplies are not removed.
    if (acc[0] == 1.5e-38f) st_agent(ws + kProbeWsSink, 1u);
  } else if (MODE > 0) {
    unsigned* flat = ws + kProbeWsFlat;       // one arrival word per segment
    unsigned* group = ws + kProbeWsGroups;    // 8 arrival words, 64 bytes apart (cumulative over segments)
    unsigned* global = ws + kProbeWsGlobal;   // cumulative group arrivals
    unsigned* go = ws + kProbeWsGo;           // [segment][group] release words
    const int grp = c & 7;
    const unsigned gsize = (unsigned)((G - 1 - grp) / 8 + 1);
    for (int s = 0; s < S; ++s) {
      unsigned spins = 0;
      for (;;) {
        unsigned m = 0xffffffffu;
        for (int w = 0; w < kW; ++w) m = min(m, lds_load(&done[w]));
        if (m >= (unsigned)s + 1 || ++spins > 4 * kSpin) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (MODE == 1) {
        if (lane == 0) add_agent(flat + s, 1u);
        wait_at_least(flat + s, (unsigned)G, error);
      } else if (MODE == 3) {
        unsigned* tags = ws + kProbeWsTags;
        if (lane < 8) st_agent(tags + lane * kProbeMaxTagGroups + c, (unsigned)s + 1);
        const unsigned* mine = tags + grp * kProbeMaxTagGroups;
        unsigned spins = 0;
        while (min_words(mine, G, lane) < (unsigned)s + 1) {
          if (ld_agent(error) != 0u) break;
          __builtin_amdgcn_s_sleep(1);
          if (++spins > kSpin) {
            if (lane == 0) st_agent(error, 1u);
            break;
          }
        }
      } else {
        unsigned old = 0;
        if (lane == 0) old = add_agent(group + grp * 16, 1u);
        old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
        unsigned* mine = go + s * 8 + grp;
        if (old % gsize == gsize - 1) {  // the last of this group to arrive at segment s
          if (lane == 0) add_agent(global, 1u);
          wait_at_least(global, 8u * (unsigned)(s + 1), error);
          if (lane == 0) st_agent(mine, 1u);
        } else {
          wait_at_least(mine, 1u, error);
        }
      }
      lds_store(&ready, (unsigned)s + 1);
    }
  }
  // The last workgroup out clears the barrier and tag words for the next
  // launch (every other workgroup has passed its last wait).
  __shared__ unsigned last;
  __syncthreads();
  if (threadIdx.x == 0) last = add_agent(ws + kProbeWsExit, 1u) == (unsigned)G - 1 ? 1u : 0u;
  __syncthreads();
  if (last) {
    if (MODE == 3)
      for (int i = threadIdx.x; i < 8 * kProbeMaxTagGroups; i += blockDim.x) st_agent(ws + kProbeWsTags + i, 0u);
    if (threadIdx.x == 0) {
      for (int i = 0; i < S; ++i) st_agent(ws + kProbeWsFlat + i, 0u);
      for (int i = 0; i < 8; ++i) st_agent(ws + kProbeWsGroups + i * 16, 0u);
      st_agent(ws + kProbeWsGlobal, 0u);
      for (int i = 0; i < 8 * S; ++i) st_agent(ws + kProbeWsGo + i, 0u);
      st_agent(ws + kProbeWsExit, 0u);
    }
  }
}

// The MFMA rate with nothing else to do: 4 waves per workgroup, each with
// 16 accumulator tiles of v_mfma_f32_32x32x16_bf16 (the prefill GEMM's
// instruction and accumulator count), 64 back-to-back MFMAs per iteration.
// The operands cycle through 8 A and 8 B fragments of pseudo-random bf16
// values in [1, 2) with random signs and mantissas, so the multipliers switch
// as they do on data (power, and with it the clock, depends on that).  A
// checksum store nobody expects keeps the work.
typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ __forceinline__ unsigned probe_hash(unsigned v) {
  v ^= v >> 16;
  v *= 0x7feb352du;
  v ^= v >> 15;
  v *= 0x846ca68bu;
  v ^= v >> 16;
  return v;
}
__device__ __forceinline__ bf16x8_t probe_fragment(unsigned seed) {
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned h = probe_hash(seed * 4u + (unsigned)i);
    // two bf16 values: sign and 7 mantissa bits random, exponent of [1, 2)
    v[i] = (0x3f80u | (h & 0x807fu)) | ((0x3f80u | ((h >> 16) & 0x807fu)) << 16);
  }
  return __builtin_bit_cast(bf16x8_t, v);
}
__global__ __launch_bounds__(256, 1) void probe_mfma_kernel(int iterations, unsigned* __restrict__ sink) {
  const unsigned id = blockIdx.x * 256u + threadIdx.x;
  bf16x8_t a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = probe_fragment(id * 16u + (unsigned)i);
    b[i] = probe_fragment(id * 16u + 8u + (unsigned)i);
  }
  f32x16_t acc[16];
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;
  for (int it = 0; it < iterations; ++it) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int t = 0; t < 16; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(t + r) & 7], b[(3 * t + r) & 7], acc[t], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < 16; ++t) s += acc[t][threadIdx.x & 15];
  if (s == 1.5e-38f) st_agent(sink, 1u);
}

}  // namespace

hipError_t launch_probe_mfma(int workgroups, int iterations, void* sink, hipStream_t stream) {
  launch_kernel(probe_mfma_kernel, dim3(workgroups), dim3(256), 0, stream, iterations, static_cast<unsigned*>(sink));
  return hipGetLastError();
}

hipError_t launch_probe_step(const void* weights, const ProbeSegments& seg, int mode, int ring, int grid,
                             void* workspace, hipStream_t stream) {
  auto* ws = static_cast<unsigned*>(workspace);
  auto* w = static_cast<const char*>(weights);
  const dim3 block((kW + 1) * 64);
  auto go = [&](auto kernel) {
    launch_kernel(kernel, dim3(grid), block, 0, stream, w, seg, ws);
    return hipGetLastError();
  };
  if (ring == 4) {
    if (mode == 0) return go(probe_step_kernel<4, 0>);
    if (mode == 1) return go(probe_step_kernel<4, 1>);
    if (mode == 2) return go(probe_step_kernel<4, 2>);
    return go(probe_step_kernel<4, 3>);
  }
  if (mode == 0) return go(probe_step_kernel<16, 0>);
  if (mode == 1) return go(probe_step_kernel<16, 1>);
  if (mode == 2) return go(probe_step_kernel<16, 2>);
  return go(probe_step_kernel<16, 3>);
}

}  // namespace lsk
