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
// (unit, segment) pairs, unit-major; workgroup g takes pairs
// [g*P/G, (g+1)*P/G).  Every CU so streams the same number of bytes of every
// projection (within one pair), whatever U is -- 160 units of o_proj and
// down_proj against 256 CUs included.
//
// Roles inside the workgroup (9 waves):
//  * 8 compute waves.  Wave w takes k-tiles 2w, 2w+1 of every segment, for
//    every row-block of the pair, so each wave's stream of 1 KB weight tiles
//    is fixed by the program.  A wave keeps kRing tile loads in flight in
//    registers and refills a slot as soon as it is multiplied, so the only
//    memory waits it has are for its own oldest weight load.  Activation
//    fragments come from LDS (staged by the control wave); accumulators of a
//    finished unit range go to LDS for the control wave.
//  * 1 control wave.  It stages each pair's activation segment into a ring
//    of LDS slots (coherent loads, after the projection's dependency is
//    met), sums the 8 compute waves' partials of each unit range in wave
//    order, and finishes units: a unit wholly inside the workgroup's range
//    is stored with its epilogue; a unit that later workgroups finish is
//    "owned" here (this workgroup has its segment 0): the owner waits for
//    their fp32 partials, adds them in workgroup order and stores; a unit
//    this workgroup enters mid-K is published as a partial for its owner.
//    After its last unit range of a projection it publishes its progress
//    word (projections completed).  A projection that depends on q starts
//    staging activations once every workgroup's progress exceeds q.  The
//    control wave never blocks on one of these while other work is ready,
//    so a workgroup always finishes what other workgroups wait for.
//
// Every sum has a fixed order (waves, then workgroups), so results are
// bitwise reproducible.  Activations, residuals, outputs, partials and
// progress cross XCDs, whose L2s are not coherent with each other, so they
// are read and written with agent-scope relaxed atomics (device-coherent
// loads and stores; no cache maintenance).  Owners wait only for later
// workgroups' partials and dependencies point to earlier projections, so
// the waits always drain with the whole grid resident (one workgroup per
// CU); every wait is bounded anyway and records an error instead of
// spinning forever.  The last workgroup out clears the progress words, and
// owners clear the partial flags they consumed, so the workspace is
// reusable by the next launch (and by graph replays) without a memset.

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
constexpr int kXBytes = 116 * 1024;                   // staged activation segments (M rows each)
constexpr int kMaxXSlots = 16;
constexpr int kRedSlots = 2;
constexpr unsigned kSpinLimit = 1u << 22;   // polls of one LDS or partial-flag wait
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
#ifdef LSK_STACK_TRACE
#define LSK_TRACE(ws_, count_, G_, g_, p_, ev_, lane_)                                                             \
  do {                                                                                                            \
    if ((lane_) == 0)                                                                                             \
      __hip_atomic_store((global_u32*)((ws_) + kStackWsBytes((count_), (G_)) / 4 +                                \
                                       ((size_t)(g_) * (count_) + (p_)) * 8 + (ev_)),                             \
                         (unsigned)__builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); \
  } while (0)
#else
#define LSK_TRACE(ws_, count_, G_, g_, p_, ev_, lane_) \
  do {                                                 \
  } while (0)
#endif

// Wave-uniform copy of a value the compiler cannot prove uniform (an LDS
// load) but that is, so branches on it stay scalar.
__device__ __forceinline__ unsigned uni(unsigned v) { return (unsigned)__builtin_amdgcn_readfirstlane((int)v); }

// LDS words shared by the waves (relaxed workgroup-scope atomics: ds ops of
// one wave execute in order, so flag/data ordering only needs the writer's
// lgkmcnt wait before the flag).
__device__ __forceinline__ unsigned lds_load(const unsigned* p) {
  return uni(__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}
__device__ __forceinline__ void lds_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(unsigned* p, unsigned v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
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
  SeqDesc seq[kStackMaxProjections];
  unsigned char xbuf[kXBytes];                         // staged activation segments
  f32x4_t red[kRedSlots][kCompute][2][64];             // compute-wave partials of a unit range
  unsigned x_ready[kMaxXSlots];                        // pair sequence number + 1 of the slot's content
  unsigned x_done[kMaxXSlots];                         // compute waves done reading the slot
  unsigned red_count[kRedSlots];                       // compute waves that wrote the slot
  unsigned red_next[kRedSlots];                        // unit-range number the slot takes next
  unsigned error;                                      // a bounded wait inside the workgroup gave up
};

// Pairs [begin, end) of workgroup g in a projection of P pairs.
__device__ __forceinline__ int range_begin(int P, int G, int g) { return (int)(((long long)P * g) / G); }

// Walks one compute wave's weight-tile sequence: projection, pair (unit,
// segment), then within the pair k-tile jk (0, 1: k-tiles 2w, 2w+1 of the
// segment) and row-block jr of the unit, jr fastest.  All counters advance
// incrementally (no division per tile).
struct Seq {
  const SeqDesc* desc;  // LDS
  int count, G, g;
  int p;          // projection (count: finished)
  int pair, end;  // current pair (index in p) and end of this workgroup's pairs
  int begin;      // first pair of this workgroup in p
  int unit, seg;  // pair = unit * NS + seg
  int jk, jr;     // k-tile of the wave's two, row-block of the unit
  int rbw, KT, NS;
  const bf16x8_t* w;

  __device__ __forceinline__ void enter(int from) {
    for (p = from; p < count; ++p) {
      const SeqDesc d = desc[p];
      const int P = d.units * (d.KT / kSeg);
      pair = range_begin(P, G, g);
      end = range_begin(P, G, g + 1);
      begin = pair;
      if (pair < end) {
        rbw = d.rbw;
        KT = d.KT;
        NS = d.KT / kSeg;
        w = d.w;
        unit = pair / NS;
        seg = pair - unit * NS;
        jk = 0;
        jr = 0;
        return;
      }
    }
  }
  __device__ __forceinline__ bool done() const { return p >= count; }
  __device__ __forceinline__ void advance() {
    if (++jr < rbw) return;
    jr = 0;
    if (++jk < kWaveTiles) return;
    jk = 0;
    if (++seg == NS) {
      seg = 0;
      ++unit;
    }
    if (++pair < end) return;
    enter(p + 1);
  }
  // This lane's 16 bytes of the current tile for compute wave `wave`.
  __device__ __forceinline__ const bf16x8_t* tile(int wave, int lane) const {
    const int kt = seg * kSeg + kWaveTiles * wave + jk;
    const int rb = unit * rbw + jr;
    return w + ((size_t)rb * KT + kt) * 64 + lane;
  }
  __device__ __forceinline__ bool pair_first() const { return jk == 0 && jr == 0; }
  __device__ __forceinline__ bool pair_last() const { return jk == kWaveTiles - 1 && jr == rbw - 1; }
  // The current pair is the last of its unit inside this workgroup's range.
  __device__ __forceinline__ bool range_last() const { return pair + 1 == end || seg + 1 == NS; }
};

// Weight ring of a compute wave.  The loads and their waits are explicit:
// with the bookkeeping branches of a tile step between a slot's load and
// its use, the compiler's own wait analysis falls back to vmcnt(0) and
// drains the ring every tile.  A compute wave issues no other vector memory
// operation, exactly one ring load per tile step, so "the oldest slot has
// landed" is exactly vmcnt(kRing - 1).  The wait names the slot's registers
// as in/out operands, so the multiply that reads them cannot be scheduled
// above it.
__device__ __forceinline__ void ring_load(bf16x8_t& dst, const bf16x8_t* p) {
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(dst) : "v"(p) : "memory");
}
__device__ __forceinline__ void ring_wait(bf16x8_t& slot) {
  static_assert(kRing == 16, "the wait count below is kRing - 1");
  asm volatile("s_waitcnt vmcnt(15)" : "+v"(slot) : : "memory");
}

// ------------------------------------------------------------ compute waves
__device__ __forceinline__ void compute_wave(const StackProgram* prog, Shared& sh, unsigned* ws, int wave, int lane) {
  Seq con{sh.seq, prog->count, (int)gridDim.x, (int)blockIdx.x};
  con.enter(0);
  Seq iss = con;
  const bf16x8_t* dummy = prog->desc[0].w + lane;  // any valid address, for loads past the end

  bf16x8_t ring[kRing];
#pragma unroll
  for (int k = 0; k < kRing; ++k) {
    ring_load(ring[k], iss.done() ? dummy : iss.tile(wave, lane));
    if (!iss.done()) iss.advance();
  }

  // Activation fragment: token (column) lane & 15, K chunk lane >> 4; the
  // tokens >= M of the 16 MFMA columns are zero (read row 0, then masked).
  const int M = prog->M;
  const int nslots = x_slots(M);
  const int slot_bytes = M * kXRow;
  const bool x_valid = (lane & 15) < M;
  const int x_lane = (x_valid ? (lane & 15) : 0) * kXRow + (lane >> 4) * 16 + kWaveTiles * wave * (kTileK * 2);
  const unsigned x_keep = x_valid ? ~0u : 0u;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  bf16x8_t xf0 = {}, xf1 = {};
  unsigned pair_seq = 0, range_seq = 0;

  // One tile: multiply ring slot k (a compile-time index, so the ring stays
  // in registers), refill it, and do the pair / unit-range bookkeeping.
  // Every step issues exactly one weight load (past the end of the sequence
  // a valid dummy address), which keeps ring_wait's count exact.
  auto tile = [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    ring_wait(ring[k]);
    if (!con.done()) {
      if (con.pair_first()) {
        const int slot = pair_seq % nslots;
        unsigned spins = 0;
        while (lds_load(&sh.x_ready[slot]) != pair_seq + 1 && lds_load(&sh.error) == 0u) {
          __builtin_amdgcn_s_sleep(1);
          if (++spins > kSpinLimit) {
            lds_store(&sh.error, 1u + (pair_seq << 8));
            break;
          }
        }
        asm volatile("" ::: "memory");
        const unsigned char* xs = sh.xbuf + slot * slot_bytes + x_lane;
        xf0 = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(xs) & x_keep);
        xf1 = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(xs + kTileK * 2) & x_keep);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) lds_add(&sh.x_done[slot], 1u);  // one count per wave
      }
      if (wave == 0 && con.pair == con.begin && con.pair_first())
        LSK_TRACE(ws, con.count, con.G, con.g, con.p, 2, lane);
      if (wave == 0 && con.pair + 1 == con.end && con.pair_last())
        LSK_TRACE(ws, con.count, con.G, con.g, con.p, 3, lane);
      const bf16x8_t xf = con.jk ? xf1 : xf0;
      if (con.jr == 0)
        acc0 = mfma16(ring[k], xf, acc0);
      else
        acc1 = mfma16(ring[k], xf, acc1);
      if (con.pair_last()) {
        if (con.range_last()) {
          const int rs = range_seq % kRedSlots;
          unsigned spins = 0;
          while (lds_load(&sh.red_next[rs]) != range_seq && lds_load(&sh.error) == 0u) {  // slot free for us
            __builtin_amdgcn_s_sleep(1);
            if (++spins > kSpinLimit) {
              lds_store(&sh.error, 3u + (range_seq << 8));
              break;
            }
          }
          asm volatile("" ::: "memory");
          sh.red[rs][wave][0][lane] = acc0;
          sh.red[rs][wave][1][lane] = acc1;
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (lane == 0) lds_add(&sh.red_count[rs], 1u);  // one count per wave
          acc0 = f32x4_t{0.f, 0.f, 0.f, 0.f};
          acc1 = f32x4_t{0.f, 0.f, 0.f, 0.f};
          ++range_seq;
        }
        ++pair_seq;
      }
      con.advance();
    }
    ring_load(ring[k], iss.done() ? dummy : iss.tile(wave, lane));
    if (!iss.done()) iss.advance();
  };
  while (!con.done()) unroll<kRing>(tile);
}

// ------------------------------------------------------------- control wave
struct ControlCtx {
  const StackProgram* prog;
  Shared* sh;
  unsigned* ws;
  unsigned* progress;   // G words
  unsigned* flags;      // count x G words
  unsigned char* parts; // count x G partial slots of kStackPartialBytes
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

__device__ __forceinline__ unsigned char* partial_slot(const ControlCtx& c, int p, int g) {
  return c.parts + ((size_t)p * c.G + g) * kStackPartialBytes;
}

__device__ __forceinline__ void store_partial(unsigned char* slot, int lane, const f32x4_t& v) {
  unsigned long long* q = reinterpret_cast<unsigned long long*>(slot + lane * 16);
  coherent_store64(q, (unsigned long long)__float_as_uint(v[0]) | ((unsigned long long)__float_as_uint(v[1]) << 32));
  coherent_store64(q + 1, (unsigned long long)__float_as_uint(v[2]) | ((unsigned long long)__float_as_uint(v[3]) << 32));
}

__device__ __forceinline__ void add_partial(f32x4_t& v, const unsigned char* slot, int lane) {
  const unsigned long long* q = reinterpret_cast<const unsigned long long*>(slot + lane * 16);
  const unsigned long long lo = coherent_load64(q), hi = coherent_load64(q + 1);
  v[0] += __uint_as_float((unsigned)lo);
  v[1] += __uint_as_float((unsigned)(lo >> 32));
  v[2] += __uint_as_float((unsigned)hi);
  v[3] += __uint_as_float((unsigned)(hi >> 32));
}

// Finish the unit range [pb, pe) of projection p (summed accumulators a0, a1).
__device__ void finish_range(const ControlCtx& c, int p, int pb, int pe, f32x4_t a0, f32x4_t a1) {
  const StackDesc& d = c.prog->desc[p];
  const int NS = d.KT / kSeg;
  const int P = d.units * NS;
  const int unit = pb / NS;
  const int unit_end = (unit + 1) * NS;
  if (pb % NS != 0) {
    // Entered mid-K: publish the partial for the owner (an earlier workgroup).
    unsigned char* slot = partial_slot(c, p, c.g);
    store_partial(slot, c.lane, a0);
    if (d.rbw == 2) store_partial(slot + 1024, c.lane, a1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (c.lane == 0) coherent_store32(c.flags + (size_t)p * c.G + c.g, 1u);
    return;
  }
  // Owner: add the partials of the later workgroups that finish the unit.
  for (int j = c.g + 1, covered = pe; covered < unit_end && j < c.G; ++j) {
    const int jb = range_begin(P, c.G, j), je = range_begin(P, c.G, j + 1);
    if (je > jb) {
      unsigned* flag = c.flags + (size_t)p * c.G + j;
      unsigned spins = 0;
      while (coherent_load32(flag) == 0u && coherent_load32(c.ws + kStackWsError) == 0u) {
        __builtin_amdgcn_s_sleep(2);
        if (++spins > kSpinLimit) {
          record_error(c, 4u, (unsigned)p, (unsigned)j, (unsigned)pb, (unsigned)pe);
          break;
        }
      }
      asm volatile("" ::: "memory");
      const unsigned char* slot = partial_slot(c, p, j);
      add_partial(a0, slot, c.lane);
      if (d.rbw == 2) add_partial(a1, slot + 1024, c.lane);
      if (c.lane == 0) coherent_store32(flag, 0u);
    }
    covered = je;
  }
  store_unit(c, d, unit, a0, a1);
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
// the LDS slots.  A batch takes the next pairs whose slot is free and whose
// dependency is met, up to kBatchRows activation rows (M per pair); all its
// row loads are issued before the first is written to LDS, so a batch costs
// one memory round trip.  (Plain coherent loads and LDS stores: an LDS DMA
// anywhere in the kernel makes the compiler wait for all vector memory
// before every LDS read, which would drain the compute waves' weight rings.)
constexpr int kBatchRows = 16;

struct XCursor {
  int xp, xpair, xend, xbegin;
  unsigned seq;
};

__device__ __forceinline__ void stager_wave(const ControlCtx& c) {
  const StackProgram* prog = c.prog;
  Shared& sh = *c.sh;
  const int G = c.G, g = c.g, count = prog->count, M = c.M, lane = c.lane;
  auto enter = [&](XCursor& x, int from) {
    for (x.xp = from; x.xp < count; ++x.xp) {
      const StackDesc& d = prog->desc[x.xp];
      const int P = d.units * (d.KT / kSeg);
      x.xpair = range_begin(P, G, g);
      x.xend = range_begin(P, G, g + 1);
      x.xbegin = x.xpair;
      if (x.xpair < x.xend) return;
    }
  };
  auto next_pair = [&](XCursor& x) {
    ++x.seq;
    if (++x.xpair >= x.xend) enter(x, x.xp + 1);
  };
  XCursor cur{0, 0, 0, 0, 0u};
  enter(cur, 0);
  unsigned idle = 0;
  int dep_ok = -1;  // projections <= dep_ok are known complete everywhere
  const int nslots = x_slots(M);
  const int slot_bytes = M * kXRow;

  // Row r of the batch that starts at cursor b: f(r, source, LDS destination).
  auto walk = [&](const XCursor& b, int nrows, auto&& f) {
    XCursor x = b;
    int m = 0;
    unroll<kBatchRows>([&](auto rc) {
      constexpr int r = decltype(rc)::value;
      if (r < nrows) {
        const StackDesc& d = prog->desc[x.xp];
        const int seg = x.xpair % (d.KT / kSeg);
        f(IntC<r>{}, d.x + (size_t)m * d.ldx + (size_t)seg * kSeg * kTileK + 8 * lane,
          sh.xbuf + (x.seq % nslots) * slot_bytes + m * kXRow + 16 * lane);
        if (++m == M) {
          m = 0;
          next_pair(x);
        }
      }
    });
  };

  while (cur.xp < count) {
    // Collect the batch.
    const XCursor start = cur;
    int nrows = 0;
    while (cur.xp < count && nrows + M <= kBatchRows) {
      const int slot = cur.seq % nslots;
      if (!(cur.seq < (unsigned)nslots || lds_load(&sh.x_done[slot]) == (unsigned)kCompute)) break;
      const StackDesc& d = prog->desc[cur.xp];
      if (d.dep > dep_ok) {
        if (!projections_done(c, d.dep)) break;
        dep_ok = d.dep;
        LSK_TRACE(c.ws, count, G, g, cur.xp, 0, lane);
      }
      nrows += M;
      next_pair(cur);
    }
    if (nrows == 0) {
      __builtin_amdgcn_s_sleep(1);
      if (give_up(c, idle, 5u, (unsigned)cur.xp, cur.seq)) return;
      continue;
    }
    idle = 0;
    u32x4_t rows[kBatchRows];
    walk(start, nrows, [&](auto rc, const __bf16* src, unsigned char*) {
      const unsigned long long* q = reinterpret_cast<const unsigned long long*>(src);
      const unsigned long long lo = coherent_load64(q), hi = coherent_load64(q + 1);
      rows[decltype(rc)::value] = u32x4_t{(unsigned)lo, (unsigned)(lo >> 32), (unsigned)hi, (unsigned)(hi >> 32)};
    });
    walk(start, nrows, [&](auto rc, const __bf16*, unsigned char* dst) {
      *reinterpret_cast<u32x4_t*>(dst) = rows[decltype(rc)::value];
    });
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    for (unsigned q = start.seq; q < cur.seq; ++q) {
      lds_store(&sh.x_done[q % nslots], 0u);
      lds_store(&sh.x_ready[q % nslots], q + 1);
    }
    if (start.xpair == start.xbegin) LSK_TRACE(c.ws, count, G, g, start.xp, 1, lane);
  }
}

// Finisher: the compute waves' partials of each unit range, in order, then
// the range's epilogue or cross-workgroup partial, and this workgroup's
// progress word after its last range of each projection.
__device__ __forceinline__ void finisher_wave(const ControlCtx& c) {
  const StackProgram* prog = c.prog;
  Shared& sh = *c.sh;
  const int G = c.G, g = c.g, count = prog->count, lane = c.lane;
  int rp = 0, rb = 0, re = 0, rend = 0;
  auto r_next_range = [&](int from_pair) {
    // First unit range starting at pair from_pair of projection rp, or the next projection's first.
    while (rp < count) {
      const StackDesc& d = prog->desc[rp];
      const int NS = d.KT / kSeg;
      const int P = d.units * NS;
      if (from_pair < 0) from_pair = range_begin(P, G, g);
      rend = range_begin(P, G, g + 1);
      if (from_pair < rend) {
        rb = from_pair;
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
  int published = 0;  // projections whose progress this workgroup has published
  while (rp < count || published < count) {
    bool did = false;
    if (rp < count) {
      const int rs = range_seq % kRedSlots;
      if (lds_load(&sh.red_count[rs]) == (unsigned)kCompute) {
        asm volatile("" ::: "memory");
        f32x4_t a0 = sh.red[rs][0][0][lane], a1 = sh.red[rs][0][1][lane];
#pragma unroll
        for (int w = 1; w < kCompute; ++w) {
          a0 += sh.red[rs][w][0][lane];
          a1 += sh.red[rs][w][1][lane];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_store(&sh.red_count[rs], 0u);
        lds_store(&sh.red_next[rs], range_seq + kRedSlots);
        finish_range(c, rp, rb, re, a0, a1);
        ++range_seq;
        r_next_range(re);
        did = true;
      }
    }
    if (published < rp) {
      LSK_TRACE(c.ws, count, G, g, rp - 1, 4, lane);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // outputs and partials stored
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
  if (threadIdx.x < kMaxXSlots) {
    sh.x_ready[threadIdx.x] = 0u;
    sh.x_done[threadIdx.x] = 0u;
  }
  if (threadIdx.x < kRedSlots) {
    sh.red_count[threadIdx.x] = 0u;
    sh.red_next[threadIdx.x] = threadIdx.x;
  }
  if (threadIdx.x == 0) sh.error = 0u;
  __syncthreads();

  if (wave < kCompute) {
    compute_wave(prog, sh, ws, wave, lane);
  } else {
    ControlCtx c{prog, &sh, ws, ws + kStackWsProgress, ws + kStackWsFlags, nullptr, (int)gridDim.x,
                 (int)blockIdx.x, lane, prog->M};
    c.parts = reinterpret_cast<unsigned char*>(ws) + kStackWsPartialsOffset(prog->count, (int)gridDim.x);
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
