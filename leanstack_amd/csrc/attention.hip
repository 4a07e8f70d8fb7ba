// Decode attention (one new token) for gfx950: the work between the QKV and
// o_proj projections of a Qwen3 decode layer, in one launch.
//
// Per (kv head j, chunk of the rows attended) one workgroup of 8 waves, from
// the raw QKV projection row (attention_rows_per_chunk: one chunk up to 128
// rows, 64-row chunks up to 512 rows, then at most 32 chunks of 128, 256,
// 384 or 512 rows):
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

// Wave-wide sum / max with the butterfly's pairing (xor 1, 2, 4, 8 inside a
// 16-lane row, then (r0 + r1) + (r2 + r3) over the rows).  The in-row steps
// are DPP moves (quad_perm [1,0,3,2], [2,3,0,1], then row_half_mirror and
// row_mirror: after the quad steps every lane of a quad holds the quad's
// value, so mirroring pairs each quad / half with the other one); partners
// combine the same two values, so every lane of a row holds identical bits.
// The rows are combined from readlanes, so all lanes get one value.
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float row_lane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xb1>(v));
  v = fmaxf(v, dpp<0x4e>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
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
  int n_q, n_kv, s_max, pos, chunks;  // chunks of attention_rows_per_chunk(pos + 1) rows
  float eps, scale;
  int grid_chunks;                    // workgroups per kv head in the grid (>= chunks)
  const int* pos_ptr;                 // device-resident pos (then cos / sin are whole tables)
};

constexpr int kCoherent = 16;  // device-coherent buffer access (partials cross XCDs)
// A buffer offset past every partial slot (num_records is at most 2^31 - 1):
// the load returns zero without a memory access.
constexpr unsigned kOutOfRange = 0x80000000u;
constexpr unsigned kRawBufferDword3 = 0x00020000u;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// One chunk's softmax state for its G heads: running max m, sum l, and the
// unnormalised P.V rows, in floats at slot offset: m[G], l[G], then acc[G][d].
__host__ __device__ constexpr unsigned partial_slot_bytes(int G) {
  return (unsigned)(G * 2 + G * kAttnHeadDim) * 4u + 12u & ~15u;
}

// The last workgroup of kv head j: M_h = max_c m_c and
// out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c, in chunk order.
// Every partial value is requested in one round (NB * 8 chunk slots per
// output; those past the last chunk load from outside the buffer's range,
// which returns zero and moves no data, and get weight 0), together with the
// (m, l) pairs, so the combine waits for memory once.
template <int G, int NB>
__device__ __forceinline__ void combine_chunks(const AttnArgs& a, __amdgpu_buffer_rsrc_t parts, unsigned first,
                                               unsigned slot_bytes, int j, float (*mx)[G], float (*lsum)[G],
                                               float (*wts)[G], float (*wl)[G]) {
  constexpr int kOut = (G * kHeadDim + kThreads - 1) / kThreads;
  constexpr int kSlots = NB * 8;
  float v[kOut][kSlots];
#pragma unroll
  for (int o = 0; o < kOut; ++o) {
    const int e = min((int)threadIdx.x + o * kThreads, G * kHeadDim - 1);
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
      // Out of range goes in the vector offset: the range check covers the
      // vector and instruction offsets, not the scalar one.
      const bool real = k < a.chunks;
      const unsigned voff = (real ? 0u : kOutOfRange) + (unsigned)(2 * G + e) * 4u;
      const unsigned base = real ? first + (unsigned)k * slot_bytes : 0u;
      v[o][k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(parts, voff, base, kCoherent));
    }
  }
  // (m, l) of chunk k, head h, to thread kG + h; weights past the last
  // chunk are 0.
  const int wk = threadIdx.x / G;
  const int wh = threadIdx.x - wk * G;
  if (wk < a.chunks) {
    const unsigned base = first + wk * slot_bytes;
    mx[wk][wh] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(parts, (unsigned)wh * 4u, base,
                                                                                  kCoherent));
    lsum[wk][wh] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(parts, (unsigned)(G + wh) * 4u,
                                                                                    base, kCoherent));
  }
  __syncthreads();
  if (wk < kSlots) {
    float m = -__builtin_huge_valf();
    for (int k = 0; k < a.chunks; ++k) m = fmaxf(m, mx[k][wh]);
    const float w = wk < a.chunks ? expf(mx[wk][wh] - m) : 0.f;
    wts[wk][wh] = w;
    wl[wk][wh] = wk < a.chunks ? w * lsum[wk][wh] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int o = 0; o < kOut; ++o) {
    const int e = threadIdx.x + o * kThreads;
    if (e >= G * kHeadDim) break;
    const int h = e / kHeadDim;
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
      num += wts[k][h] * v[o][k];
      den += wl[k][h];
    }
    a.out[(size_t)(j * G) * kHeadDim + e] = static_cast<__bf16>(num / den);
  }
}

// DYN: pos is read from device memory (a.pos_ptr), cos / sin are the whole
// position tables ([s_max][d/2]), and the chunk size and count follow from
// pos here; the grid holds the most chunks max_seq_len can need and the
// workgroups past this pos's count leave at once.  A pos outside
// [0, s_max) leaves every buffer untouched.
template <int G, int NU, bool DYN>
__global__ __launch_bounds__(kThreads) void decode_attention_kernel(AttnArgs args) {
  static_assert(G >= 1 && G <= 16, "q heads per kv head are the MFMA B columns");
  constexpr int kGroups = NU;              // 16-row groups per wave
  constexpr int kRows = 16 * kWaves * NU;  // rows per workgroup at most: 128 NU
  constexpr int kMaxChunks = kAttnMaxChunks;
  AttnArgs a = args;
  if constexpr (DYN) {
    const int pos = *args.pos_ptr;
    if (pos < 0 || pos >= a.s_max) return;
    a.pos = pos;
    a.cos += (size_t)pos * (kHeadDim / 2);
    a.sin += (size_t)pos * (kHeadDim / 2);
  }
  // Rows per chunk (at most kRows: the launch picks NU for the largest chunk
  // it can meet) and the chunk count, as the host computes them.
  const int rows = attention_rows_per_chunk(a.pos + 1);
  a.chunks = (a.pos + rows) / rows;  // ceil((pos + 1) / rows)
  const int j = blockIdx.x / a.grid_chunks;
  const int ci = blockIdx.x - j * a.grid_chunks;
  if (ci >= a.chunks) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int L = a.pos + 1;
  const int row0 = ci * rows;
  // Wave w owns the chunk's 16-row groups w, w + 8, w + 16, ...: group u of
  // the wave starts at chunk row lb(u) = 16 (w + 8u).  Groups past the last
  // row are skipped, so short contexts cost little and the waves share the
  // rows evenly.
  auto lb = [&](int u) { return 16 * (wave + kWaves * u); };
  const bool has_new = a.pos >= row0 && a.pos < row0 + rows;

  __shared__ __align__(16) __bf16 qs[16][kHeadDim];     // rotated q heads; rows >= G are zero
  __shared__ __align__(16) __bf16 kv_new[2][kHeadDim];  // this token's rotated k and its v
  __shared__ __align__(16) float sc[G][kRows];          // scores, then exp(s - m)
  __shared__ __align__(16) float part[kWaves][G][kHeadDim];
  __shared__ float stat[2][G];                          // chunk max, chunk sum
  __shared__ float cmax[kMaxChunks][G];                 // combine: chunk maxima m_c
  __shared__ float lsum[kMaxChunks][G];                 // combine: chunk sums l_c
  __shared__ float wts[kMaxChunks][G];                  // combine: e^(m_c - M)
  __shared__ float wl[kMaxChunks][G];                   // combine: e^(m_c - M) l_c
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
      if (t < a.pos && lb(u) < rows)
        v = *reinterpret_cast<const bf16x8_t*>(kbase + (size_t)t * kHeadDim + 32 * kt + 8 * g);
      kf[u][kt] = v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tv = row0 + lb(u) + 4 * i + g;
      bf16x8_t v = {};
      if (tv < a.pos && lb(u) < rows) v = *reinterpret_cast<const bf16x8_t*>(vbase + (size_t)tv * kHeadDim + 8 * c);
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
    if (lb(u) >= rows || row0 + lb(u) >= L) break;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[u][kt], qf[kt], acc, 0, 0, 0);
    if (c < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[c][lb(u) + 4 * g + i] = acc[i] * a.scale;
    }
  }
  __syncthreads();

  // ---- chunk softmax state per head over its filled rows n (up to
  // kRows / 64 per lane, summed in row order within a lane, then across
  // lanes); the rows past the last are never read again.
  const int n = min(rows, L - row0);
  for (int h = wave; h < G; h += kWaves) {
    float sv[kRows / 64];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int u = 0; u < kRows / 64; ++u) {
      if (64 * u >= n) break;
      sv[u] = lane + 64 * u < n ? sc[h][lane + 64 * u] : -__builtin_huge_valf();
      mx = fmaxf(mx, sv[u]);
    }
    const float m = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < kRows / 64; ++u) {
      if (64 * u >= n) break;
      const float e = lane + 64 * u < n ? expf(sv[u] - m) : 0.f;
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
  // for dims 8c .. 8c+7, then the four row phases g are added as
  // (g0 + g1) + (g2 + g3) by a reduce-scatter (each exchange sends half of
  // what a lane holds, so lane (g, c) ends with a quarter of the 8G sums),
  // and the waves' sums in wave order.
  float acc8[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc8[h][e] = 0.f;
#pragma unroll
  for (int u = 0; u < kGroups; ++u) {
    if (lb(u) >= rows || row0 + lb(u) >= L) break;
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
  constexpr int kHalf = 4 * G;  // of the 8G values (flat index q = 8h + e)
  const bool odd = g & 1, high = g >> 1;
  float half[kHalf];
#pragma unroll
  for (int q = 0; q < kHalf; ++q) {
    const float lo = acc8[q / 8][q % 8], hi = acc8[(q + kHalf) / 8][(q + kHalf) % 8];
    half[q] = (odd ? hi : lo) + __shfl_xor(odd ? lo : hi, 16);
  }
  // lane (g, c) now holds flat indices kHalf * odd + q, q < kHalf
  float quarter[kHalf / 2];
#pragma unroll
  for (int q = 0; q < kHalf / 2; ++q) {
    const float lo = half[q], hi = half[q + kHalf / 2];
    quarter[q] = (high ? hi : lo) + __shfl_xor(high ? lo : hi, 32);
  }
  const int q0 = kHalf * odd + (kHalf / 2) * high;
#pragma unroll
  for (int q = 0; q < kHalf / 2; ++q) part[wave][(q0 + q) / 8][8 * c + (q0 + q) % 8] = quarter[q];
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

  const unsigned first = (unsigned)(j * a.chunks) * slot_bytes;
  if (a.chunks <= 8) {
    combine_chunks<G, 1>(a, parts, first, slot_bytes, j, cmax, lsum, wts, wl);
  } else if (a.chunks <= 16) {
    combine_chunks<G, 2>(a, parts, first, slot_bytes, j, cmax, lsum, wts, wl);
  } else if (a.chunks <= 24) {
    combine_chunks<G, 3>(a, parts, first, slot_bytes, j, cmax, lsum, wts, wl);
  } else {
    combine_chunks<G, 4>(a, parts, first, slot_bytes, j, cmax, lsum, wts, wl);
  }
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + j, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int G, int NU, bool DYN = false>
hipError_t launch_gu(const AttnArgs& a, hipStream_t stream) {
  launch_kernel(decode_attention_kernel<G, NU, DYN>, dim3(a.n_kv * a.grid_chunks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template <int G>
hipError_t launch_dyn(const AttnArgs& a, int nu, hipStream_t stream) {
  switch (nu) {
    case 1:
      return launch_gu<G, 1, true>(a, stream);
    case 2:
      return launch_gu<G, 2, true>(a, stream);
    case 3:
      return launch_gu<G, 3, true>(a, stream);
    case 4:
      return launch_gu<G, 4, true>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

template <int G>
hipError_t launch_g(const AttnArgs& a, int nu, hipStream_t stream) {
  switch (nu) {
    case 1:
      return launch_gu<G, 1>(a, stream);
    case 2:
      return launch_gu<G, 2>(a, stream);
    case 3:
      return launch_gu<G, 3>(a, stream);
    case 4:
      return launch_gu<G, 4>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

int attention_chunk_rows(int rows) { return attention_rows_per_chunk(rows); }

size_t attention_workspace_bytes(int n_q, int n_kv, int max_seq_len) {
  const int group = n_q / n_kv;
  return kAttnPartialsOffset + (size_t)n_kv * attention_most_chunks(max_seq_len) * partial_slot_bytes(group);
}

namespace {

AttnArgs common_args(const void* qkv, int n_q, int n_kv, const void* q_norm_w, const void* k_norm_w, float eps,
                     const void* cos, const void* sin, void* k_cache, void* v_cache, int s_max, float scale,
                     void* out, void* workspace, size_t ws_bytes) {
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
  a.pos = 0;
  a.chunks = 1;
  a.grid_chunks = 1;
  a.pos_ptr = nullptr;
  a.eps = eps;
  a.scale = scale;
  auto* ws = static_cast<unsigned char*>(workspace);
  a.counters = reinterpret_cast<unsigned*>(ws);
  a.partials = ws != nullptr ? ws + kAttnPartialsOffset : nullptr;
  const size_t pb = ws_bytes > kAttnPartialsOffset ? ws_bytes - kAttnPartialsOffset : 0;
  a.partial_bytes = (unsigned)(pb < 0x7fffffffu ? pb : 0x7fffffffu);
  return a;
}

}  // namespace

hipError_t launch_decode_attention(const void* qkv, int n_q, int n_kv, const void* q_norm_w, const void* k_norm_w,
                                   float eps, const void* cos, const void* sin, void* k_cache, void* v_cache,
                                   int s_max, int pos, float scale, void* out, void* workspace, size_t ws_bytes,
                                   hipStream_t stream) {
  AttnArgs a = common_args(qkv, n_q, n_kv, q_norm_w, k_norm_w, eps, cos, sin, k_cache, v_cache, s_max, scale, out,
                           workspace, ws_bytes);
  a.pos = pos;
  const int rows = attention_chunk_rows(pos + 1);
  const int nu = (rows + 127) / 128;  // 16-row groups per wave: 8 waves x 16 rows x nu cover the chunk
  a.chunks = (pos + 1 + rows - 1) / rows;
  a.grid_chunks = a.chunks;
  switch (n_q / n_kv) {
    case 1:
      return launch_g<1>(a, nu, stream);
    case 2:
      return launch_g<2>(a, nu, stream);
    case 4:
      return launch_g<4>(a, nu, stream);
    case 8:
      return launch_g<8>(a, nu, stream);
    default:
      return hipErrorInvalidValue;
  }
}

int attention_grid_chunks(int max_seq_len) { return attention_most_chunks(max_seq_len); }

hipError_t launch_decode_attention_at(const void* qkv, int n_q, int n_kv, const void* q_norm_w, const void* k_norm_w,
                                      float eps, const void* cos_table, const void* sin_table, void* k_cache,
                                      void* v_cache, int s_max, const int* pos_device, float scale, void* out,
                                      void* workspace, size_t ws_bytes, hipStream_t stream) {
  AttnArgs a = common_args(qkv, n_q, n_kv, q_norm_w, k_norm_w, eps, cos_table, sin_table, k_cache, v_cache, s_max,
                           scale, out, workspace, ws_bytes);
  a.pos_ptr = pos_device;
  a.grid_chunks = attention_grid_chunks(s_max);
  // Chunks never exceed the size max_seq_len rows need (the rule grows with
  // the rows attended), so that size fixes the kernel's groups per wave.
  const int nu = (attention_chunk_rows(s_max) + 127) / 128;
  switch (n_q / n_kv) {
    case 1:
      return launch_dyn<1>(a, nu, stream);
    case 2:
      return launch_dyn<2>(a, nu, stream);
    case 4:
      return launch_dyn<4>(a, nu, stream);
    case 8:
      return launch_dyn<8>(a, nu, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace lsk
