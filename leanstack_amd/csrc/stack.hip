// Persistent decode-step kernel: a whole sequence of projections (e.g. the
// 36 layers x {QKV, o_proj, gate_up + SiLU*up, down} of a decode or verify
// step at M <= 16) in ONE launch, streaming weights from HBM without a gap at
// projection boundaries.
//
// Why: each projection is only 21-100 MB, 3-14 us of HBM time, so separate
// launches pay every kernel's ramp-up and tail (2-3 us per launch).  Here one
// workgroup per CU walks its share of every projection in order, and the
// weight stream of the next projection is already in flight while the
// current one finishes: weights never depend on activations.
//
// Work split.  A projection of U units (16 weight rows, or a 32-row gate/up
// pair for SiLU*up) and K = NS segments of 512 is a list of U*NS
// (unit, segment) pairs, unit-major; workgroup g takes the whole units
// [g*U/G, (g+1)*U/G), so every unit's sum stays inside one workgroup.  When
// U < G (o_proj and down_proj: 160 units), the workgroups without a unit go
// straight on to the next projection's weights.
//
// Roles inside the workgroup (10 waves):
//  * 8 compute waves.  Wave w takes k-tiles 2w, 2w+1 of every segment, for
//    every row-block of the unit, so each wave's stream of 1 KB weight tiles
//    is fixed by the program.  A wave keeps kRing tile loads in flight in
//    registers and refills a slot as soon as it is multiplied, so the only
//    memory waits it has are for its own oldest weight load.  Activation
//    fragments come from LDS (staged by the stager); the accumulators of a
//    finished unit go to LDS for the finisher.
//  * The stager stages each pair's activation segment into a ring of LDS
//    slots (device-coherent loads when the input is produced inside the
//    launch), once every workgroup's progress shows the projection's
//    dependency complete.
//  * The finisher sums the 8 compute waves' accumulators of each unit in
//    wave order, stores the unit with its epilogue and, after a projection's
//    last unit, publishes this workgroup's progress word (projections
//    completed).
// Neither control wave blocks on a wait while work that others wait for is
// ready, so a workgroup always finishes what other workgroups wait for.
//
// Every sum has a fixed order, so results are bitwise reproducible.
// Activations, residuals, outputs and progress cross XCDs, whose L2s are not
// coherent with each other, so they are read and written with agent-scope
// relaxed atomics (device-coherent loads and stores; no cache maintenance).
// Dependencies point to earlier projections and the whole grid is resident
// (one workgroup per CU), so the waits always drain; every wait is bounded
// anyway and records an error instead of spinning forever.  The last
// workgroup out clears the progress words, so the workspace is reusable by
// the next launch (and by graph replays) without a memset.

#include <hip/hip_runtime.h>

#include "lsk_internal.h"

namespace lsk {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kCompute = kStackComputeWaves;          // 8
constexpr int kThreads = (kCompute + 2) * 64;         // + stager and finisher waves
constexpr int kSeg = kStackSegTiles;                  // 16 k-tiles (512 K) per segment
constexpr int kWaveTiles = kSeg / kCompute;           // 2 k-tiles per compute wave per segment
constexpr int kRing = 16;                             // weight tiles in flight per compute wave
constexpr int kXRow = kSeg * kTileK * 2 + 16;         // LDS bytes per activation row (+16: bank skew)
constexpr int kXBytes = 104 * 1024;                   // staged activation segments (M rows each)
constexpr int kMaxXSlots = 64;
constexpr int kRedSlots = 2;
constexpr unsigned kSpinLimit = 1u << 22;   // polls of one LDS wait
constexpr unsigned kIdleLimit = 1u << 20;   // control-wave rounds without progress


template <int I>
struct IntC {
  static constexpr int value = I;
};
// f(IntC<0>{}), ..., f(IntC<N-1>{}) in order.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void unroll(F&& f) {
  if constexpr (I < N) {
    f(IntC<I>{});
    unroll<N, I + 1>(f);
  }
}
typedef __attribute__((address_space(1))) unsigned long long global_u64;
typedef __attribute__((address_space(1))) unsigned global_u32;

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}


__device__ __forceinline__ unsigned long long coherent_load64(const void* p) {
  return __hip_atomic_load((const global_u64*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void coherent_store64(void* p, unsigned long long v) {
  __hip_atomic_store((global_u64*)(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned coherent_load32(const unsigned* p) {
  return __hip_atomic_load((const global_u32*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void coherent_store32(unsigned* p, unsigned v) {
  __hip_atomic_store((global_u32*)(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Optional event timestamps (build with -DLSK_STACK_TRACE): word
// (g * count + p) * 8 + event of a buffer placed right after the workspace
// receives the constant-clock time of the event for workgroup g, projection p.
// Events: 0 dependency seen met, 6 first batch sized, 7 its loads landed,
// 1 first activations staged, 2 first multiply, 3 last multiply, 4 last unit
// stored, 5 progress published.
#ifdef LSK_STACK_TRACE
#define LSK_TRACE(ws_, count_, G_, g_, p_, ev_, lane_)                                                             \
  do {                                                                                                            \
    if ((lane_) == 0)                                                                                             \
      __hip_atomic_store((global_u32*)((ws_) + kStackWsBytes((count_), (G_)) / 4 +                                \
                                       ((size_t)(g_) * (count_) + (p_)) * 8 + (ev_)),                             \
                         (unsigned)__builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); \
  } while (0)
// Per compute wave: 0, cycles in the activation wait, in the accumulator-slot
// wait, and in total, at word (G*count*8) + (g*8 + wave)*4 + i.
#define LSK_STALL_BEGIN() const unsigned long long stall_t0_ = __builtin_amdgcn_s_memtime()
#define LSK_STALL_END(acc_) (acc_) += __builtin_amdgcn_s_memtime() - stall_t0_
#else
#define LSK_TRACE(ws_, count_, G_, g_, p_, ev_, lane_) \
  do {                                                 \
  } while (0)
#define LSK_STALL_BEGIN() \
  do {                    \
  } while (0)
#define LSK_STALL_END(acc_) \
  do {                      \
  } while (0)
#endif

// Wave-uniform copy of a value the compiler cannot prove uniform (an LDS
// load) but that is, so branches on it stay scalar.
__device__ __forceinline__ unsigned uni(unsigned v) { return (unsigned)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// LDS words shared by the waves (relaxed workgroup-scope atomics: ds ops of
// one wave execute in order, so flag/data ordering only needs the writer's
// lgkmcnt wait before the flag).
__device__ __forceinline__ unsigned lds_load(const unsigned* p) {
  return uni(__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}
__device__ __forceinline__ void lds_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Activation slot i holds the M rows of one pair's segment at
// xbuf + i * M * kXRow; there are min(kMaxXSlots, kXBytes / (M * kXRow)).
__host__ __device__ constexpr int x_slots(int M) {
  return kXBytes / (M * kXRow) < kMaxXSlots ? kXBytes / (M * kXRow) : kMaxXSlots;
}

// What the compute waves need of a projection, copied to LDS at launch so
// their cursors never issue a vector load (which would disturb the weight
// ring's wait count).
struct SeqDesc {
  const bf16x8_t* w;
  int units;
  short KT, rbw;
};

struct Shared {
  StackDesc desc[kStackMaxProjections];                // the program, for the stager and finisher
  SeqDesc seq[kStackMaxProjections];
  unsigned char xbuf[kXBytes];                         // staged activation segments
  unsigned char xzero[kXRow];                          // zeros: the fragment of tokens >= M
  f32x4_t red[kRedSlots][kCompute][2][64];             // compute-wave partials of a unit range
  unsigned x_staged;                                   // pairs whose activations are in their slot
  unsigned x_used[kCompute];                           // pairs each compute wave has read
  unsigned red_done[kCompute];                         // unit ranges each compute wave has written
  unsigned red_freed;                                  // unit ranges the finisher has read
  unsigned error;                                      // a bounded wait inside the workgroup gave up
};

// Projection p's descriptor from the LDS copy, every word made wave-uniform
// (control waves branch and address on it; a scalar-cache miss on the
// program in global memory costs a memory round trip under the weight stream).
__device__ __forceinline__ StackDesc lds_desc(const Shared& sh, int p) {
  static_assert(sizeof(StackDesc) % 4 == 0, "descriptor copied as 32-bit words");
  constexpr int kWords = sizeof(StackDesc) / 4;
  unsigned w[kWords];
  const unsigned* src = reinterpret_cast<const unsigned*>(&sh.desc[p]);
#pragma unroll
  for (int i = 0; i < kWords; ++i) w[i] = uni(src[i]);
  return __builtin_bit_cast(StackDesc, w);
}

// First pair of workgroup g in a projection of `units` units of NS pairs:
// workgroup g takes whole units [units*g/G, units*(g+1)/G), so no unit's sum
// is split between workgroups (units * G < 2^32: packed weights are under
// 4 GiB and G <= kStackMaxGrid).
__device__ __forceinline__ int range_begin(int units, int NS, int G, int g) {
  return (int)((unsigned)units * (unsigned)g / (unsigned)G) * NS;
}

// Raw buffer resource over `bytes` bytes at `base` (wave-uniform).
constexpr int kNonTemporal = 2;  // buffer-load cache policy: streamed once
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)0x00020000u);
}

// A compute wave's weight-tile stream, one ring round (kRing tiles) at a
// time.  Per projection it is the wave's tiles of the workgroup's pairs in
// order (a pair: k-tiles jk = 0, 1 of the wave in one segment of a unit, for
// each row-block jr of the unit, jr fastest), padded with dummy tiles (tile 0
// of the projection, never multiplied) to whole rounds, so every projection
// starts at ring slot 0.  next() returns one round: lane t < kRing holds the
// byte offset of the round's tile t, and the resource of its projection.
// The lanes compute the offsets in parallel, once per round; the tile steps
// only read them.
struct Round {
  unsigned off;
  __amdgpu_buffer_rsrc_t rsrc;
};

// Pairs [b, e) of workgroup g in projection d (0 pairs: b == e).
struct Share {
  int b, e, R, NS, KT;
  __device__ __forceinline__ Share(const SeqDesc& d, int G, int g) {
    KT = uni((int)d.KT);
    NS = KT / kSeg;
    R = uni((int)d.rbw);
    const int units = uni(d.units);
    b = range_begin(units, NS, G, g);
    e = range_begin(units, NS, G, g + 1);
  }
};

struct Planner {
  const SeqDesc* desc;  // LDS
  int count, G, g, wave, lane;
  int p;                 // projection being issued; count: past the end (dummies)
  int round, rounds, b, pairs, R, NS, KT;
  __amdgpu_buffer_rsrc_t rsrc;

  __device__ __forceinline__ void enter(int from) {
    for (p = from; p < count; ++p) {
      const SeqDesc d = desc[p];
      const Share s(d, G, g);
      if (s.b < s.e) {
        R = s.R;
        KT = s.KT;
        NS = s.NS;
        b = s.b;
        pairs = s.e - s.b;
        rounds = (pairs * 2 * R + kRing - 1) / kRing;
        round = 0;
        rsrc = weight_rsrc(d.w, (unsigned)uni(d.units) * (unsigned)(R * KT) * 1024u);
        return;
      }
    }
  }
  __device__ __forceinline__ Round next() {
    Round r{0u, rsrc};
    if (p < count) {
      const int T = round * kRing + (lane & (kRing - 1));
      const int pair = T >> R;  // 2R tiles per pair, R = 1 or 2
      const int j = T & (2 * R - 1);
      const int jr = j & (R - 1), jk = j >> (R - 1);
      if (pair < pairs) {
        const unsigned P = (unsigned)(b + pair);
        const unsigned unit = P / (unsigned)NS;
        const unsigned seg = P - unit * (unsigned)NS;
        r.off = ((unit * R + jr) * (unsigned)KT + seg * kSeg + kWaveTiles * wave + jk) * 1024u;
      }
      if (++round == rounds) enter(p + 1);
    }
    return r;
  }
};

__device__ __forceinline__ bf16x8_t ring_load(const Round& r, int k, unsigned lane16) {
  return __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                          r.rsrc, lane16, (unsigned)__builtin_amdgcn_readlane((int)r.off, k),
                                          kNonTemporal));
}

// ------------------------------------------------------------ compute waves
// Each round multiplies the kRing tiles in the ring and refills every slot
// with the planner's next round, so kRing tile loads stay in flight.  One
// loop serves every projection (the row-block count R only selects which
// accumulator and fragment a slot's multiply uses), so the ring keeps one
// register assignment throughout.
__device__ __forceinline__ void compute_wave(const StackProgram* prog, Shared& sh, unsigned* ws, int wave, int lane) {
  const int count = prog->count, G = gridDim.x, g = blockIdx.x;
  Planner plan{sh.seq, count, G, g, wave, lane};
  plan.rsrc = weight_rsrc(sh.seq[0].w, 1024u);
  plan.enter(0);
  const unsigned lane16 = (unsigned)lane * 16u;

  bf16x8_t ring[kRing];
  {
    const Round r0 = plan.next();
    unroll<kRing>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      ring[k] = ring_load(r0, k, lane16);
    });
  }

  // Activation fragment: token (column) lane & 15, K chunk lane >> 4.  Lanes
  // of tokens >= M read a zero row instead.
  const int M = prog->M;
  const int nslots = x_slots(M);
  const unsigned slot_bytes = (unsigned)(M * kXRow);
  const bool x_valid = (lane & 15) < M;
  const unsigned x_col = (unsigned)((lane >> 4) * 16 + kWaveTiles * wave * (kTileK * 2));
  const unsigned x_lane = (unsigned)(uintptr_t)sh.xbuf + (unsigned)((lane & 15) * kXRow) + x_col;
  const unsigned x_zero = (unsigned)(uintptr_t)sh.xzero + x_col;
  unsigned pair_seq = 0, range_seq = 0;
  unsigned x_avail = 0, red_avail = kRedSlots;  // pairs staged, unit ranges with a free slot (as last seen)
  int slot = 0;
  unsigned slot_off = 0;
#ifdef LSK_STACK_TRACE
  unsigned long long st_x = 0, st_red = 0;
  const unsigned long long st_start = __builtin_amdgcn_s_memtime();
#endif

  // Consumer cursor: projection cp, its pairs, the pair done next, its segment.
  int cp = -1, R = 1, NS = 1, pairs = 0, done = 0, seg = 0, rounds = 0, round = 0;
  auto consume_enter = [&]() {
    for (++cp; cp < count; ++cp) {
      const Share s(sh.seq[cp], G, g);
      if (s.b < s.e) {
        R = s.R;
        NS = s.NS;
        pairs = s.e - s.b;
        seg = s.b % s.NS;
        done = 0;
        rounds = (pairs * 2 * R + kRing - 1) / kRing;
        round = 0;
        return;
      }
    }
  };
  consume_enter();

  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  bf16x8_t xf0 = {}, xf1 = {};
  bool real = false;
  while (cp < count) {
    const Round nr = plan.next();
    const bool r2 = R == 2;
    unroll<kRing>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if constexpr (k % 2 == 0) {
        if (!r2 || k % 4 == 0) {  // a pair starts: its activation fragments
          real = done < pairs;
          if (real) {
            if (pair_seq >= x_avail) {
              unsigned spins = 0;
              LSK_STALL_BEGIN();
#pragma clang loop unroll(disable)
              while ((x_avail = lds_load(&sh.x_staged)) <= pair_seq) {
                if (lds_load(&sh.error) != 0u) break;
                __builtin_amdgcn_s_sleep(1);
                if (++spins > kSpinLimit) {
                  lds_store(&sh.error, 1u + (pair_seq << 8));
                  break;
                }
              }
              LSK_STALL_END(st_x);
            }
            asm volatile("" ::: "memory");
            const unsigned xa = x_valid ? x_lane + slot_off : x_zero;
            const auto* xs = reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(xa);
            xf0 = __builtin_bit_cast(bf16x8_t, xs[0]);
            xf1 = __builtin_bit_cast(bf16x8_t, xs[kTileK * 2 / 16]);
            // The LDS executes one wave's operations in order, so the stager
            // (which reuses the slot only after seeing this count) cannot
            // overwrite the fragments before these reads have taken them.
            asm volatile("" ::: "memory");
            lds_store(&sh.x_used[wave], pair_seq + 1);
            if (wave == 0 && done == 0) LSK_TRACE(ws, count, G, g, cp, 2, lane);
          }
        }
      }
      if (real) {
        if (r2) {  // tiles (jr, jk) = (k & 1, (k >> 1) & 1) of the pair
          if constexpr (k % 2 == 0)
            acc0 = mfma16(ring[k], ((k >> 1) & 1) ? xf1 : xf0, acc0);
          else
            acc1 = mfma16(ring[k], ((k >> 1) & 1) ? xf1 : xf0, acc1);
        } else {  // tiles jk = k & 1 of one row-block
          acc0 = mfma16(ring[k], (k & 1) ? xf1 : xf0, acc0);
        }
      }
      ring[k] = ring_load(nr, k, lane16);
      if constexpr (k % 2 == 1) {
        if ((!r2 || k % 4 == 3) && real) {  // a pair ends
          if (done + 1 == pairs || seg + 1 == NS) {  // ... and with it a unit range of this workgroup
            if (wave == 0 && done + 1 == pairs) LSK_TRACE(ws, count, G, g, cp, 3, lane);
            const int rs = range_seq % kRedSlots;
            if (range_seq >= red_avail) {  // slot rs still holds range range_seq - kRedSlots
              unsigned spins = 0;
              LSK_STALL_BEGIN();
#pragma clang loop unroll(disable)
              while ((red_avail = lds_load(&sh.red_freed) + kRedSlots) <= range_seq) {
                if (lds_load(&sh.error) != 0u) break;
                __builtin_amdgcn_s_sleep(1);
                if (++spins > kSpinLimit) {
                  lds_store(&sh.error, 3u + (range_seq << 8));
                  break;
                }
              }
              LSK_STALL_END(st_red);
            }
            asm volatile("" ::: "memory");
            sh.red[rs][wave][0][lane] = acc0;
            sh.red[rs][wave][1][lane] = acc1;
            asm volatile("" ::: "memory");
            lds_store(&sh.red_done[wave], range_seq + 1);  // after the partials, in LDS order
            acc0 = f32x4_t{0.f, 0.f, 0.f, 0.f};
            acc1 = f32x4_t{0.f, 0.f, 0.f, 0.f};
            ++range_seq;
          }
          ++pair_seq;
          ++done;
          if (++seg == NS) seg = 0;
          slot_off += slot_bytes;
          if (++slot == nslots) {
            slot = 0;
            slot_off = 0;
          }
        }
      }
    });
    if (++round == rounds) consume_enter();
  }
#ifdef LSK_STACK_TRACE
  if (lane == 0) {
    unsigned* st = ws + kStackWsBytes(count, G) / 4 + (size_t)G * count * 8 + (g * 8 + wave) * 4;
    const unsigned long long total = __builtin_amdgcn_s_memtime() - st_start;
    st[0] = 0u;
    st[1] = (unsigned)(st_x >> 8);
    st[2] = (unsigned)(st_red >> 8);
    st[3] = (unsigned)(total >> 8);
  }
#endif
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last round's (dummy) loads
}

// ------------------------------------------------------------- control wave
struct ControlCtx {
  const StackProgram* prog;
  Shared* sh;
  unsigned* ws;
  unsigned* progress;   // G words
  int G, g, lane, M;
};

// The first bounded wait of a launch to give up claims the detail record
// (workspace words kStackWsDetail..+7): workgroup + 1, which wait gave up,
// and the control wave's cursors, for lsk_stack_error's caller to inspect.
__device__ __forceinline__ void record_error(const ControlCtx& c, unsigned code, unsigned a = 0, unsigned b = 0,
                                             unsigned d = 0, unsigned e = 0, unsigned f = 0) {
  unsigned expected = 0u;
  if (__hip_atomic_compare_exchange_strong((global_u32*)(c.ws + kStackWsDetail), &expected, (unsigned)c.g + 1u,
                                           __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
    const unsigned v[6] = {code, a, b, d, e, f};
    for (int i = 0; i < 6; ++i) coherent_store32(c.ws + kStackWsDetail + 1 + i, v[i]);
  }
  coherent_store32(c.ws + kStackWsError, 1u);
}

// Have all workgroups completed projections 0..q?  (One poll, no wait.)
__device__ __forceinline__ bool projections_done(const ControlCtx& c, int q) {
  // Up to 4 * 64 workgroups per poll, all loads issued before the compares.
  bool ok = true;
  for (int base = 0; base < c.G; base += 4 * 64) {
    unsigned v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = base + i * 64 + c.lane;
      v[i] = coherent_load32(c.progress + (idx < c.G ? idx : c.G - 1));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) ok &= v[i] > (unsigned)q;
  }
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// Epilogue of unit `unit` of projection d from the summed accumulators.
// Lane l holds output rows 4(l>>4)+i (i < 4) of the unit for token l & 15.
__device__ __forceinline__ void store_unit(const ControlCtx& c, const StackDesc& d, int unit, const f32x4_t& a0,
                                           const f32x4_t& a1) {
  const int m = c.lane & 15;
  if (m >= c.M) return;
  const int n = unit * kTileRows + 4 * (c.lane >> 4);  // output column (intermediate index for SiLU*up)
  float v[4];
  if (d.epi == static_cast<int>(Epilogue::kSiluMul)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = silu_mul_bf16(a0[i], a1[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = bf16_round(a0[i]);
    if (d.epi == static_cast<int>(Epilogue::kResidualAdd)) {
      const unsigned long long r = coherent_load64(d.res + (size_t)m * d.ldr + n);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += __builtin_bit_cast(float, (unsigned)((r >> (16 * i)) & 0xffffu) << 16);
    }
  }
  const unsigned long long packed = (unsigned long long)bf16_bits(v[0]) | ((unsigned long long)bf16_bits(v[1]) << 16) |
                                    ((unsigned long long)bf16_bits(v[2]) << 32) |
                                    ((unsigned long long)bf16_bits(v[3]) << 48);
  coherent_store64(d.y + (size_t)m * d.ldy + n, packed);
}

// The summed accumulators of unit `unit` of projection p (every unit range
// is a whole unit: workgroups take whole units).
__device__ __forceinline__ void finish_unit(const ControlCtx& c, int p, int unit, f32x4_t a0, f32x4_t a1) {
  store_unit(c, lds_desc(*c.sh, p), unit, a0, a1);
}

// A bounded wait of a control wave has gone on too long, or another wave or
// workgroup gave up: record it once and release every wave of the workgroup.
__device__ __forceinline__ bool give_up(const ControlCtx& c, unsigned& idle, unsigned code, unsigned a, unsigned b) {
  if (++idle <= kIdleLimit && !((idle & 1023u) == 0u && (coherent_load32(c.ws + kStackWsError) != 0u ||
                                                         lds_load(&c.sh->error) != 0u)))
    return false;
  const unsigned lerr = lds_load(&c.sh->error);
  record_error(c, lerr != 0u ? (0x100u | lerr) : (idle > kIdleLimit ? code : 7u), a, b);
  lds_store(&c.sh->error, 1u);
  return true;
}

// Stager: activation segments of this workgroup's pairs, in pair order, into
// the LDS slots.  A batch is the next run of one projection's pairs whose
// slots are free (once the projection's dependency is met), up to kBatchRows
// activation rows (M per pair); all its row loads are issued before the
// first is written to LDS, so a batch costs one memory round trip, and the
// projection's descriptor stays in registers for the whole run.  (Plain
// loads and LDS stores: an LDS DMA anywhere in the kernel makes the compiler
// wait for all vector memory before every LDS read, which would drain the
// compute waves' weight rings.)
constexpr int kBatchRows = 16;

__device__ __forceinline__ void stager_wave(const ControlCtx& c) {
  const StackProgram* prog = c.prog;
  Shared& sh = *c.sh;
  const int G = c.G, g = c.g, count = prog->count, M = c.M, lane = c.lane;
  const int nslots = x_slots(M);
  const unsigned slot_bytes = (unsigned)(M * kXRow);
  const int batch_pairs = kBatchRows / M;  // >= 1: M <= 16

  // Projection xp being staged: its pairs [xpair, xend), activation rows.
  int xp = 0, xpair = 0, xend = 0, xbegin = 0, NS = 1, ldx = 0, dep = -1;
  const __bf16* xbase = nullptr;
  auto enter = [&](int from) {
    for (xp = from; xp < count; ++xp) {
      const StackDesc d = lds_desc(sh, xp);
      NS = d.KT / kSeg;
      xpair = range_begin(d.units, NS, G, g);
      xend = range_begin(d.units, NS, G, g + 1);
      if (xpair < xend) {
        xbegin = xpair;
        xbase = d.x;
        ldx = d.ldx;
        dep = d.dep;
        return;
      }
    }
  };
  enter(0);

  // Pairs every compute wave has read.
  auto used_min = [&]() {
    unsigned v[kCompute];
#pragma unroll
    for (int w = 0; w < kCompute; ++w) v[w] = __hip_atomic_load(&sh.x_used[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    unsigned m = v[0];
#pragma unroll
    for (int w = 1; w < kCompute; ++w) m = v[w] < m ? v[w] : m;
    return uni(m);
  };
  unsigned seq = 0, used = 0, idle = 0;
  int dep_ok = -1;  // projections <= dep_ok are known complete everywhere
  int slot = 0;     // seq % nslots

  while (xp < count) {
    if (dep > dep_ok) {
      if (!projections_done(c, dep)) {
        __builtin_amdgcn_s_sleep(1);
        if (give_up(c, idle, 5u, (unsigned)xp, seq)) return;
        continue;
      }
      dep_ok = dep;
      LSK_TRACE(c.ws, count, G, g, xp, 0, lane);
    }
    // Slot of pair seq + i is free once every wave has read pair seq + i - nslots.
    if (seq >= used + (unsigned)nslots) used = used_min();
    const int free_slots = (int)(used + (unsigned)nslots - seq);
    if (free_slots <= 0) {
      __builtin_amdgcn_s_sleep(1);
      if (give_up(c, idle, 5u, (unsigned)xp, seq)) return;
      continue;
    }
    idle = 0;
    int n = xend - xpair;
    n = n < free_slots ? n : free_slots;
    n = n < batch_pairs ? n : batch_pairs;
    const int nrows = n * M;
    if (xpair == xbegin) LSK_TRACE(c.ws, count, G, g, xp, 6, lane);

    // Row r of the batch: pair xpair + r / M, activation row r % M.
    u32x4_t rows[kBatchRows];
    {
      int m = 0, seg = xpair % NS;
      const __bf16* src = xbase + (size_t)seg * kSeg * kTileK + 8 * lane;
      unroll<kBatchRows>([&](auto rc) {
        constexpr int r = decltype(rc)::value;
        if (r < nrows) {
          const __bf16* row = src + (size_t)m * ldx;
          if (dep >= 0) {
            // Produced inside this launch by other workgroups: device-coherent loads.
            const unsigned long long* q = reinterpret_cast<const unsigned long long*>(row);
            const unsigned long long lo = coherent_load64(q), hi = coherent_load64(q + 1);
            rows[r] = u32x4_t{(unsigned)lo, (unsigned)(lo >> 32), (unsigned)hi, (unsigned)(hi >> 32)};
          } else {
            // Ready at launch and never written by the program: plain cached loads.
            rows[r] = *reinterpret_cast<const u32x4_t*>(row);
          }
          if (++m == M) {
            m = 0;
            if (++seg == NS) seg = 0;
            src = xbase + (size_t)seg * kSeg * kTileK + 8 * lane;
          }
        }
      });
    }
#ifdef LSK_STACK_TRACE
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (xpair == xbegin) LSK_TRACE(c.ws, count, G, g, xp, 7, lane);
#endif
    {
      int m = 0, sl = slot;
      unsigned char* dst = sh.xbuf + (unsigned)sl * slot_bytes + 16 * lane;
      unroll<kBatchRows>([&](auto rc) {
        constexpr int r = decltype(rc)::value;
        if (r < nrows) {
          *reinterpret_cast<u32x4_t*>(dst + m * kXRow) = rows[r];
          if (++m == M) {
            m = 0;
            if (++sl == nslots) sl = 0;
            dst = sh.xbuf + (unsigned)sl * slot_bytes + 16 * lane;
          }
        }
      });
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    seq += (unsigned)n;
    lds_store(&sh.x_staged, seq);
    if (xpair == xbegin) LSK_TRACE(c.ws, count, G, g, xp, 1, lane);
    slot = (slot + n) % nslots;
    xpair += n;
    if (xpair == xend) enter(xp + 1);
  }
}

// Finisher: the compute waves' accumulators of each unit, in order, then
// the unit's epilogue and store, and this workgroup's progress word after
// its last unit of each projection.
__device__ __forceinline__ void finisher_wave(const ControlCtx& c) {
  const StackProgram* prog = c.prog;
  Shared& sh = *c.sh;
  const int G = c.G, g = c.g, count = prog->count, lane = c.lane;
  int rp = 0, rb = 0, re = 0, rend = 0, rns = 1;
  auto r_next_range = [&](int from_pair) {
    // First unit range starting at pair from_pair of projection rp, or the next projection's first.
    while (rp < count) {
      const StackDesc d = lds_desc(sh, rp);
      const int NS = d.KT / kSeg;
      if (from_pair < 0) from_pair = range_begin(d.units, NS, G, g);
      rend = range_begin(d.units, NS, G, g + 1);
      if (from_pair < rend) {
        rb = from_pair;
        rns = NS;
        const int unit_end = (from_pair / NS + 1) * NS;
        re = unit_end < rend ? unit_end : rend;
        return;
      }
      ++rp;
      from_pair = -1;
    }
  };
  r_next_range(-1);
  unsigned range_seq = 0, idle = 0;
  // Unit ranges every compute wave has written.
  auto written_min = [&]() {
    unsigned v[kCompute];
#pragma unroll
    for (int w = 0; w < kCompute; ++w)
      v[w] = __hip_atomic_load(&sh.red_done[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    unsigned m = v[0];
#pragma unroll
    for (int w = 1; w < kCompute; ++w) m = v[w] < m ? v[w] : m;
    return uni(m);
  };
  unsigned written = 0;
  int published = 0;  // projections whose progress this workgroup has published
  while (rp < count || published < count) {
    bool did = false;
    if (rp < count) {
      const int rs = range_seq % kRedSlots;
      if (written <= range_seq) written = written_min();
      if (written > range_seq) {
        asm volatile("" ::: "memory");
        f32x4_t a0 = sh.red[rs][0][0][lane], a1 = sh.red[rs][0][1][lane];
#pragma unroll
        for (int w = 1; w < kCompute; ++w) {
          a0 += sh.red[rs][w][0][lane];
          a1 += sh.red[rs][w][1][lane];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_store(&sh.red_freed, range_seq + 1);
        finish_unit(c, rp, rb / rns, a0, a1);
        ++range_seq;
        r_next_range(re);
        did = true;
      }
    }
    if (published < rp) {
      LSK_TRACE(c.ws, count, G, g, rp - 1, 4, lane);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // outputs stored
      published = rp;
      if (lane == 0) coherent_store32(c.progress + g, (unsigned)published);
      LSK_TRACE(c.ws, count, G, g, rp - 1, 5, lane);
      did = true;
    }
    if (did) {
      idle = 0;
    } else {
      __builtin_amdgcn_s_sleep(1);
      if (give_up(c, idle, 8u, (unsigned)rp | ((unsigned)published << 16), range_seq)) return;
    }
  }
}

__global__ __launch_bounds__(kThreads, 1) void decode_stack_kernel(const StackProgram* __restrict__ prog,
                                                                    unsigned* __restrict__ ws) {
  __shared__ Shared sh;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (prog->magic != kStackMagic || prog->M < 1 || prog->M > kTileRows || prog->count > kStackMaxProjections) {
    if (threadIdx.x == 0) coherent_store32(ws + kStackWsError, 2u);
    return;
  }
  for (int i = threadIdx.x; i < prog->count; i += kThreads) {
    const StackDesc& d = prog->desc[i];
    sh.seq[i] = SeqDesc{d.w, d.units, (short)d.KT, (short)d.rbw};
  }
  {
    constexpr int kWords = sizeof(StackDesc) / 4;
    const unsigned* src = reinterpret_cast<const unsigned*>(prog->desc);
    unsigned* dst = reinterpret_cast<unsigned*>(sh.desc);
    for (int i = threadIdx.x; i < prog->count * kWords; i += kThreads) dst[i] = src[i];
  }
  if (threadIdx.x < kCompute) {
    sh.x_used[threadIdx.x] = 0u;
    sh.red_done[threadIdx.x] = 0u;
  }
  if (threadIdx.x == 0) {
    sh.x_staged = 0u;
    sh.red_freed = 0u;
    sh.error = 0u;
  }
  for (int i = threadIdx.x; i < kXRow / 4; i += kThreads) reinterpret_cast<unsigned*>(sh.xzero)[i] = 0u;
  __syncthreads();

  if (wave < kCompute) {
    compute_wave(prog, sh, ws, wave, lane);
  } else {
    ControlCtx c{prog, &sh, ws, ws + kStackWsProgress, (int)gridDim.x, (int)blockIdx.x, lane, prog->M};
    if (wave == kCompute)
      stager_wave(c);
    else
      finisher_wave(c);
  }

  // Last workgroup out clears the progress words for the next launch.
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned* exit_count = ws + kStackWsExit;
    const unsigned old = __hip_atomic_fetch_add(exit_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gridDim.x - 1) {
      for (int i = 0; i < (int)gridDim.x; ++i) coherent_store32(ws + kStackWsProgress + i, 0u);
      coherent_store32(exit_count, 0u);
    }
  }
}

}  // namespace

size_t stack_lds_bytes() { return 0; }

const void* stack_kernel_symbol() { return reinterpret_cast<const void*>(&decode_stack_kernel); }

int stack_threads() { return kThreads; }

hipError_t launch_decode_stack(const StackProgram* prog, unsigned* ws, int grid, size_t lds_bytes,
                               hipStream_t stream) {
  decode_stack_kernel<<<dim3(grid), dim3(kThreads), lds_bytes, stream>>>(prog, ws);
  return hipGetLastError();
}

}  // namespace lsk
