// Decode attention (one new token) for gfx950: the work between the QKV and
// o_proj projections of a Qwen3 decode layer, in one launch.
//
// Per (kv head j, 512-row chunk of the cache) one workgroup of 8 waves, from
// the raw QKV projection row:
//   1. q heads jG..jG+G-1 and k head j: RMSNorm over head_dim with the q / k
//      norm weights, then rotate-half RoPE with this position's cos / sin
//      (src/leanstack/runtime/qwen_explicit.py:796-806, :690-716), in the
//      reference's bf16 rounding chain: bf16(x*r*w) for the norm (torch's
//      fused F.rms_norm order (x*r)*w), and a bf16 rounding after every
//      multiply and every add / subtract of the rotation;
//   2. k and v of the token appended to the static cache at row `pos`
//      (src/leanstack/runtime/kv_cache.py:222-245, batch 1);
//   3. softmax(q K^T * scale) V over rows 0..pos of kv head j for its G q
//      heads (F.scaled_dot_product_attention with enable_gqa, no mask:
//      qwen_explicit.py:894-912), scores and softmax in fp32, output bf16.
//
// Scores run on MFMA: 16 cache rows x 32 dims of K form the A operand
// (one 16-byte load per lane, straight from the row-major cache) and the G
// bf16 q heads, padded to 16 columns, the B operand.  P.V runs on the VALU,
// each wave over its 16-row groups with lane l owning dims 2l, 2l+1, and the
// waves' partial sums are added in wave order.  A context longer than one
// chunk leaves each chunk's (max, sum, unnormalised P.V) in the workspace;
// the workgroup that arrives last for kv head j combines the chunks in chunk
// order and re-arms the head's counter.  Every sum has a fixed order, so
// results are bitwise reproducible.  The new row is read from LDS, not back
// from the cache it was just written to.

#include <hip/hip_runtime.h>

#include "lsk_internal.h"

namespace lsk {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = kAttnHeadDim;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;

__device__ __forceinline__ float bf16r(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

// 1 / sqrt(ss / n + eps) with the mean rounded before eps is added, as
// torch's rms_norm computes it (contraction would fuse the two into an fma).
__device__ __forceinline__ float inv_rms(float ss, int n, float eps) {
#pragma clang fp contract(off)
  return 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
}

// One half of the rotate-half RoPE pair, a*c - b*s (sign = -1) or
// a*c + b*s (sign = +1), each product rounded to bf16 before the sum, as the
// reference's separate bf16 tensor ops round them.  Contraction is off: with
// it the compiler fuses the first product into the sum as one fma and skips
// that product's rounding.
__device__ __forceinline__ __bf16 rope_half(float a, float b, float c, float s, float sign) {
#pragma clang fp contract(off)
  return static_cast<__bf16>(bf16r(a * c) + sign * bf16r(b * s));
}

// Butterfly sum / max: partners add the same two values, so every lane ends
// with the identical result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

struct AttnArgs {
  const __bf16* qkv;       // [n_q*d | n_kv*d | n_kv*d]
  const __bf16* q_norm_w;  // [d]
  const __bf16* k_norm_w;  // [d]
  const __bf16* cos;       // [d/2], this position
  const __bf16* sin;       // [d/2]
  __bf16* k_cache;         // [n_kv][s_max][d], this layer
  __bf16* v_cache;
  __bf16* out;             // [n_q*d]
  unsigned* counters;      // workspace: one arrival counter per kv head
  unsigned char* partials; // workspace: one AttnPartial slot per (kv head, chunk)
  unsigned partial_bytes;  // bytes of all slots of this launch
  int n_q, n_kv, s_max, pos, chunks;
  float eps, scale;
};

constexpr int kCoherent = 16;  // device-coherent buffer access (partials cross XCDs)
constexpr unsigned kRawBufferDword3 = 0x00020000u;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// One chunk's softmax state for its G heads: running max m, sum l, and the
// unnormalised P.V rows, in floats at slot offset: m[G], l[G], then acc[G][d].
__host__ __device__ constexpr unsigned partial_slot_bytes(int G) {
  return (unsigned)(G * 2 + G * kAttnHeadDim) * 4u + 12u & ~15u;
}

template <int G>
__global__ __launch_bounds__(kThreads) void decode_attention_kernel(AttnArgs a) {
  static_assert(G >= 1 && G <= 16, "q heads per kv head are the MFMA B columns");
  constexpr int kRows = kAttnChunkRows;  // rows per workgroup
  constexpr int kGroups = kRows / 16 / kWaves;  // 16-row groups per wave: 4
  constexpr int kMaxChunks = kAttnMaxChunks;
  const int j = blockIdx.x / a.chunks;
  const int ci = blockIdx.x - j * a.chunks;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int L = a.pos + 1;
  const int row0 = ci * kRows;
  // Wave w owns the chunk's 16-row groups w, w + 8, w + 16, w + 24: group u
  // of the wave starts at chunk row lb(u) = 16 (w + 8u).  Groups past the last
  // row are skipped, so short contexts cost little and the waves share the
  // rows evenly.
  auto lb = [&](int u) { return 16 * (wave + kWaves * u); };
  const bool has_new = a.pos >= row0 && a.pos < row0 + kRows;

  __shared__ __align__(16) __bf16 qs[16][kHeadDim];     // rotated q heads; rows >= G are zero
  __shared__ __align__(16) __bf16 kv_new[2][kHeadDim];  // this token's rotated k and its v
  __shared__ __align__(16) float sc[G][kRows];          // scores, then exp(s - m)
  __shared__ __align__(16) float part[kWaves][G][kHeadDim];
  __shared__ float stat[2][G];                          // chunk max, chunk sum
  __shared__ float wts[kMaxChunks][G];                  // combine: chunk maxima, then e^(m_c - M)
  __shared__ float lsum[kMaxChunks][G];                 // combine: chunk sums
  __shared__ float denom[G];
  __shared__ int last;

  // ---- inputs of this wave's prologue items, loaded before the cache rows
  // so that the norms and rotations run while the rows stream in.  Item
  // i = wave + 8u: i < G is q head jG+i, i == G the k head j (only in the
  // chunk holding row pos).  Loads are unconditional (items past the last
  // read a q head again and store nothing): a load used only under a branch
  // may be sunk into it, behind the cache-row loads.  Lane l: dims l, l + 64.
  constexpr int kItems = (G + kWaves) / kWaves;  // ceil((G + 1) / kWaves)
  float px0[kItems], px1[kItems], pw0[kItems], pw1[kItems];
#pragma unroll
  for (int u = 0; u < kItems; ++u) {
    const int i = wave + kWaves * u;
    const bool is_k = i == G;
    const int src_head = is_k ? a.n_q + j : j * G + (i < G ? i : G - 1);
    const __bf16* src = a.qkv + (size_t)src_head * kHeadDim;
    const __bf16* nw = is_k ? a.k_norm_w : a.q_norm_w;
    px0[u] = static_cast<float>(src[lane]);
    px1[u] = static_cast<float>(src[lane + 64]);
    pw0[u] = static_cast<float>(nw[lane]);
    pw1[u] = static_cast<float>(nw[lane + 64]);
  }
  const float cs = static_cast<float>(a.cos[lane]);
  const float sn = static_cast<float>(a.sin[lane]);
  const __bf16* vsrc = a.qkv + ((size_t)a.n_q + a.n_kv + j) * kHeadDim;
  const __bf16 v_new0 = vsrc[lane];
  const __bf16 v_new1 = vsrc[lane + 64];
  __builtin_amdgcn_sched_barrier(0);

  // ---- cache rows of this wave (they do not depend on q).  K as MFMA A
  // fragments: group u, lane (g, c) = row lb(u) + c, dims 32kt + 8g .. +7.
  // V: lane (g, c) = dims 8c .. 8c+7 of rows lb(u) + 4i + g.  Row pos is this
  // token's (from LDS below); rows past it are not read.
  const __bf16* kbase = a.k_cache + (size_t)j * a.s_max * kHeadDim;
  const __bf16* vbase = a.v_cache + (size_t)j * a.s_max * kHeadDim;
  bf16x8_t kf[kGroups][4];
  bf16x8_t vf[kGroups][4];
#pragma unroll
  for (int u = 0; u < kGroups; ++u) {
    const int t = row0 + lb(u) + c;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      bf16x8_t v = {};
      if (t < a.pos) v = *reinterpret_cast<const bf16x8_t*>(kbase + (size_t)t * kHeadDim + 32 * kt + 8 * g);
      kf[u][kt] = v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tv = row0 + lb(u) + 4 * i + g;
      bf16x8_t v = {};
      if (tv < a.pos) v = *reinterpret_cast<const bf16x8_t*>(vbase + (size_t)tv * kHeadDim + 8 * c);
      vf[u][i] = v;
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the prologue items: RMSNorm, RoPE; k and v appended to the caches.
#pragma unroll
  for (int u = 0; u < kItems; ++u) {
    const int i = wave + kWaves * u;
    const float r = inv_rms(wave_sum(px0[u] * px0[u] + px1[u] * px1[u]), kHeadDim, a.eps);
    const float n0 = bf16r((px0[u] * r) * pw0[u]);
    const float n1 = bf16r((px1[u] * r) * pw1[u]);
    const __bf16 o0 = rope_half(n0, n1, cs, sn, -1.f);
    const __bf16 o1 = rope_half(n1, n0, cs, sn, 1.f);
    if (i < G) {
      qs[i][lane] = o0;
      qs[i][lane + 64] = o1;
    } else if (i == G && has_new) {
      kv_new[0][lane] = o0;
      kv_new[0][lane + 64] = o1;
      kv_new[1][lane] = v_new0;
      kv_new[1][lane + 64] = v_new1;
      __bf16* kc = a.k_cache + ((size_t)j * a.s_max + a.pos) * kHeadDim;
      __bf16* vc = a.v_cache + ((size_t)j * a.s_max + a.pos) * kHeadDim;
      kc[lane] = o0;
      kc[lane + 64] = o1;
      vc[lane] = v_new0;
      vc[lane + 64] = v_new1;
    }
  }
  for (int e = threadIdx.x; e < (16 - G) * kHeadDim; e += kThreads) qs[G + e / kHeadDim][e % kHeadDim] = __bf16(0.f);
  __syncthreads();

  // ---- this token's row pos, if it falls in one of this wave's groups.
  // (Unrolled selects: a runtime index would put kf / vf in scratch memory.)
  if (has_new) {
    const bf16x8_t vn = *reinterpret_cast<const bf16x8_t*>(&kv_new[1][8 * c]);
#pragma unroll
    for (int u = 0; u < kGroups; ++u) {
      const int d = a.pos - row0 - lb(u);
      if (d < 0 || d >= 16) continue;
      if (c == d) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kf[u][kt] = *reinterpret_cast<const bf16x8_t*>(&kv_new[0][32 * kt + 8 * g]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (d == 4 * i + g) vf[u][i] = vn;
    }
  }

  // ---- scores: output lane (g, c) holds rows lb(u) + 4g .. +3 of head c.
  bf16x8_t qf[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) qf[kt] = *reinterpret_cast<const bf16x8_t*>(&qs[c][32 * kt + 8 * g]);
#pragma unroll
  for (int u = 0; u < kGroups; ++u) {
    if (row0 + lb(u) >= L) break;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[u][kt], qf[kt], acc, 0, 0, 0);
    if (c < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[c][lb(u) + 4 * g + i] = acc[i] * a.scale;
    }
  }
  __syncthreads();

  // ---- chunk softmax state per head over its rows (kRows / 64 per lane,
  // summed in row order within a lane, then across lanes); rows past the
  // last get weight 0 (their score slots were never written).
  for (int h = wave; h < G; h += kWaves) {
    float sv[kRows / 64];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < kRows / 64; ++u) {
      sv[u] = row0 + lane + 64 * u < L ? sc[h][lane + 64 * u] : -__builtin_huge_valf();
      mx = fmaxf(mx, sv[u]);
    }
    const float m = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < kRows / 64; ++u) {
      const float e = row0 + lane + 64 * u < L ? expf(sv[u] - m) : 0.f;
      sc[h][lane + 64 * u] = e;
      sum += e;
    }
    const float l = wave_sum(sum);
    if (lane == 0) {
      stat[0][h] = m;
      stat[1][h] = l;
    }
  }
  __syncthreads();

  // ---- P.V over this wave's groups: lane (g, c) sums rows lb(u) + 4i + g
  // for dims 8c .. 8c+7, then the four row phases g are added (butterfly)
  // and the waves' sums in wave order.
  float acc8[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc8[h][e] = 0.f;
#pragma unroll
  for (int u = 0; u < kGroups; ++u) {
    if (row0 + lb(u) >= L) break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tl = lb(u) + 4 * i + g;  // row within the chunk
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pr = sc[h][tl];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc8[h][e] += pr * static_cast<float>(vf[u][i][e]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc8[h][e];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc8[h][e] = v;
    }
  }
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) part[wave][h][8 * c + e] = acc8[h][e];
  }
  __syncthreads();

  if (a.chunks == 1) {
    for (int e = threadIdx.x; e < G * kHeadDim; e += kThreads) {
      const int h = e / kHeadDim;
      const int d = e - h * kHeadDim;
      float s = part[0][h][d];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) s += part[w][h][d];
      a.out[(size_t)(j * G + h) * kHeadDim + d] = static_cast<__bf16>(s / stat[1][h]);
    }
    return;
  }

  // ---- several chunks: publish (m, l, acc) to slot (j, ci) with
  // device-coherent stores; the last chunk of kv head j to arrive combines
  // all of them in chunk order (so the result does not depend on which
  // one), writes the output and re-arms the counter.  Nothing waits.
  const __amdgpu_buffer_rsrc_t parts =
      __builtin_amdgcn_make_buffer_rsrc(a.partials, (short)0, (int)a.partial_bytes, (int)kRawBufferDword3);
  const unsigned slot_bytes = partial_slot_bytes(G);
  const unsigned slot = (unsigned)(j * a.chunks + ci) * slot_bytes;
  for (int e = threadIdx.x; e < G * kHeadDim; e += kThreads) {
    const int h = e / kHeadDim;
    const int d = e - h * kHeadDim;
    float s = part[0][h][d];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += part[w][h][d];
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, s), parts, (unsigned)(2 * G + e) * 4u, slot,
                                          kCoherent);
  }
  if (threadIdx.x < 2 * G) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, stat[threadIdx.x / G][threadIdx.x % G]), parts,
                                          threadIdx.x * 4u, slot, kCoherent);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    last = __hip_atomic_fetch_add(a.counters + j, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (unsigned)a.chunks - 1;
  }
  __syncthreads();
  if (!last) return;

  // Combine: M_h = max_c m_c, out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c.
  // All (m, l) pairs come in one round of loads; the partial values in
  // rounds of 8 chunks (loads past the last chunk are skipped).
  const unsigned first = (unsigned)(j * a.chunks) * slot_bytes;
  for (int e = threadIdx.x; e < a.chunks * G; e += kThreads) {
    const int k = e / G;
    const int h = e - k * G;
    const unsigned base = first + k * slot_bytes;
    wts[k][h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(parts, (unsigned)h * 4u, base,
                                                                                 kCoherent));
    lsum[k][h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(parts, (unsigned)(G + h) * 4u, base,
                                                                                  kCoherent));
  }
  __syncthreads();
  if (threadIdx.x < G) {
    const int h = threadIdx.x;
    float mx = -__builtin_huge_valf();
    for (int k = 0; k < a.chunks; ++k) mx = fmaxf(mx, wts[k][h]);
    float den = 0.f;
    for (int k = 0; k < a.chunks; ++k) {
      const float w = expf(wts[k][h] - mx);
      wts[k][h] = w;
      den += w * lsum[k][h];
    }
    denom[h] = den;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < G * kHeadDim; e += kThreads) {
    const int h = e / kHeadDim;
    float num = 0.f;
    for (int k = 0; k < a.chunks; k += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = k + u < a.chunks ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                parts, (unsigned)(2 * G + e) * 4u,
                                                                first + (k + u) * slot_bytes, kCoherent))
                                : 0.f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k + u < a.chunks) num += wts[k + u][h] * v[u];
    }
    a.out[(size_t)(j * G) * kHeadDim + e] = static_cast<__bf16>(num / denom[h]);
  }
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + j, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int G>
hipError_t launch_g(const AttnArgs& a, hipStream_t stream) {
  decode_attention_kernel<G><<<dim3(a.n_kv * a.chunks), dim3(kThreads), 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace

size_t attention_workspace_bytes(int n_q, int n_kv, int max_seq_len) {
  const int group = n_q / n_kv;
  const size_t chunks = ((size_t)max_seq_len + kAttnChunkRows - 1) / kAttnChunkRows;
  return kAttnPartialsOffset + (size_t)n_kv * chunks * partial_slot_bytes(group);
}

bool attention_group_supported(int group) { return group == 1 || group == 2 || group == 4 || group == 8; }

hipError_t launch_decode_attention(const void* qkv, int n_q, int n_kv, const void* q_norm_w, const void* k_norm_w,
                                   float eps, const void* cos, const void* sin, void* k_cache, void* v_cache,
                                   int s_max, int pos, float scale, void* out, void* workspace, size_t ws_bytes,
                                   hipStream_t stream) {
  AttnArgs a;
  a.qkv = static_cast<const __bf16*>(qkv);
  a.q_norm_w = static_cast<const __bf16*>(q_norm_w);
  a.k_norm_w = static_cast<const __bf16*>(k_norm_w);
  a.cos = static_cast<const __bf16*>(cos);
  a.sin = static_cast<const __bf16*>(sin);
  a.k_cache = static_cast<__bf16*>(k_cache);
  a.v_cache = static_cast<__bf16*>(v_cache);
  a.out = static_cast<__bf16*>(out);
  a.n_q = n_q;
  a.n_kv = n_kv;
  a.s_max = s_max;
  a.pos = pos;
  a.chunks = (pos + 1 + kAttnChunkRows - 1) / kAttnChunkRows;
  a.eps = eps;
  a.scale = scale;
  auto* ws = static_cast<unsigned char*>(workspace);
  a.counters = reinterpret_cast<unsigned*>(ws);
  a.partials = ws != nullptr ? ws + kAttnPartialsOffset : nullptr;
  const size_t pb = ws_bytes > kAttnPartialsOffset ? ws_bytes - kAttnPartialsOffset : 0;
  a.partial_bytes = (unsigned)(pb < 0x7fffffffu ? pb : 0x7fffffffu);
  switch (n_q / n_kv) {
    case 1:
      return launch_g<1>(a, stream);
    case 2:
      return launch_g<2>(a, stream);
    case 4:
      return launch_g<4>(a, stream);
    case 8:
      return launch_g<8>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace lsk
