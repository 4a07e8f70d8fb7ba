// Internal declarations shared by the C-ABI layer (abi.cpp) and the gfx950
// kernel translation units (decode.hip, gemm.hip).  Not part of the ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "lsk_host.h"

namespace lsk {


// Prefill GEMM block tile: BN weight rows x BM tokens x BK.
constexpr int kGemmBN = 128;
constexpr int kGemmBM = 128;
constexpr int kGemmBK = 64;

// Split-K prefill workspace (gemm.hip): word 0 is the error word (nonzero
// after a bounded wait gave up), an arrival and a departure word per split
// output block from kSkFlagsOffset, one fp32 256x256 partial block per split
// workgroup from kSkPartialsOffset.  Zero-filled before first use; every
// launch leaves the flags zero.
constexpr size_t kSkFlagsOffset = 256;
constexpr size_t kSkPartialsOffset = 8192;
constexpr size_t kSkPartialBytes = 256 * 256 * 4;
constexpr int kSkMaxGrid = (int)((kSkPartialsOffset - kSkFlagsOffset) / 4);
constexpr unsigned kSkSpinLimit = 1u << 22;

// Projections of kDecodeMaxM < M <= kSkinnyMaxM rows (skinny.hip).
constexpr int kSkinnyMaxM = 128;
constexpr int kSkinnyWaves = 8;
// Split-K arrival counters live in the prefill workspace's flag words (each
// call leaves them zero), partial slots from kSkPartialsOffset.
constexpr int kSkinnyMaxGroups = (int)((kSkPartialsOffset - kSkFlagsOffset) / 4);

// Persistent decode-step kernel (stack.hip).
constexpr int kStackComputeWaves = 8;  // compute waves per workgroup (+1 control wave)
constexpr int kStackSegTiles = 16;     // k-tiles per K segment of a work pair (K % 512 == 0)
constexpr int kStackMaxProjections = 256;
constexpr unsigned kStackMagic = 0x4c534b32u;
// Workspace (32-bit words): error word, exit counter, the detail record of
// the first failed wait, and one progress word per workgroup.
constexpr int kStackWsError = 0;      // nonzero after a bounded wait gave up
constexpr int kStackWsExit = 1;       // workgroups finished (reset by the last)
constexpr int kStackWsDetail = 8;     // 8 words: first failed wait (workgroup + 1, code, state)
constexpr int kStackWsProgress = 64;  // G words: projections completed by each workgroup
constexpr int kStackWsWords = 2048;
constexpr int kStackMaxGrid = kStackWsWords - kStackWsProgress;
__host__ __device__ constexpr size_t kStackWsBytes(int count, int G) {
  return (void)count, (void)G, (size_t)kStackWsWords * 4;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Device arithmetic shared by the kernel translation units.

__device__ __forceinline__ float bf16_round(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

__device__ __forceinline__ unsigned short bf16_bits(float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}

// SiLU(g) * u with the rounding chain of the reference: the gate_up product is
// a bf16 tensor, F.silu returns bf16, and the product is rounded to bf16
// (src/leanstack/runtime/qwen_explicit.py:828-830, :942-948).  sigmoid(g) =
// 1 / (1 + 2^(-g log2 e)) on the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32, 1 ulp each): with the rounding of -g log2 e the float32 result
// is within ~2^-17 relative of the exact one for |g| < 88.7, far inside the
// 2^-9 half-ulp of the bf16 it is rounded to, so the two differ by one bf16
// ulp only where the exact value lies that close to a rounding boundary.
// v_rcp_f32 flushes a subnormal result, so a denominator above 2^96 (g below
// -66.5) is scaled by 2^-32 before it and the quotient by 2^-32 after.
// Below g = -88.7, exp(-g) overflows float32 and the result is -0, as the
// float32 formula g / (1 + exp(-g)) gives there.
__device__ __forceinline__ float silu_mul_bf16(float g_acc, float u_acc) {
  const float g = bf16_round(g_acc);
  const float u = bf16_round(u_acc);
  const float d = 1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
  const float sc = d > 0x1p96f ? 0x1p-32f : 1.0f;
  const float s = bf16_round(sc * (g * __builtin_amdgcn_rcpf(d * sc)));
  return bf16_round(s * u);
}

// One projection of a stack program, as the kernel reads it (64 bytes).
struct StackDesc {
  const bf16x8_t* w;
  const __bf16* x;
  __bf16* y;
  const __bf16* res;
  int KT, ldx, ldy, ldr;
  int epi;    // Epilogue
  int rbw;    // row-blocks per unit: 1, or 2 for a SiLU gate/up pair
  int units;  // N / (16 * rbw)
  int dep;    // -1, or: every projection <= dep completes before this one reads x / residual
};

struct StackProgram {
  int count;
  int M;
  unsigned magic;
  int pad[13];
  StackDesc desc[1];  // `count` entries follow the header
};

hipError_t launch_decode_stack(const StackProgram* prog, unsigned* ws, int grid, size_t lds_bytes,
                               hipStream_t stream);
size_t stack_lds_bytes();
const void* stack_kernel_symbol();
int stack_threads();

// Argmax partial written by each lm_head workgroup: (score, index).
struct ArgmaxPartial {
  float score;
  int index;
};

enum class Epilogue : int { kNone = 0, kSiluMul = 1, kResidualAdd = 2 };

// Decode / verify launch (M <= 16).  All pointers are device pointers that
// the caller has validated.  Returns the hipError_t of the launch.
hipError_t launch_decode_linear(const void* w, int N, int K, const void* x, int M, int ldx,
                                void* y, int ldy, Epilogue epi, const void* residual, int ldr,
                                hipStream_t stream);

// The same with an RMSNorm of each x row in front of the projection
// (norm_w: bf16 [K], 16-byte aligned).
hipError_t launch_decode_rmsnorm_linear(const void* w, int N, int K, const void* x, int M, int ldx,
                                        const void* norm_w, float eps, void* y, int ldy, Epilogue epi,
                                        const void* residual, int ldr, hipStream_t stream);

// Decode attention (attention.hip).  The rows attended are split into
// chunks by attention_rows_per_chunk (one chunk up to 128 rows, then at most
// kAttnMaxChunks chunks of at least kAttnSplitRows rows), one workgroup per
// (kv head, chunk).
// Workspace: one arrival counter per kv head (kAttnMaxKvHeads words), then
// from kAttnPartialsOffset one partial slot per (kv head, chunk).
// Zero-filled before first use; every launch leaves the counters zero.
constexpr size_t kAttnPartialsOffset = kAttnMaxKvHeads * 4;

// Rows per chunk when `rows` rows are attended (attention_rows_per_chunk).
int attention_chunk_rows(int rows);

// Workspace bytes for n_kv kv heads of n_q / n_kv q heads and up to
// max_seq_len rows (needed when more than kAttnMinChunkRows rows are
// attended).
size_t attention_workspace_bytes(int n_q, int n_kv, int max_seq_len);

// One new token of one layer: q/k norms, RoPE, KV-cache append at row `pos`,
// GQA attention over rows 0..pos.  Pointers validated by the caller.
hipError_t launch_decode_attention(const void* qkv, int n_q, int n_kv, const void* q_norm_w, const void* k_norm_w,
                                   float eps, const void* cos, const void* sin, void* k_cache, void* v_cache,
                                   int s_max, int pos, float scale, void* out, void* workspace, size_t ws_bytes,
                                   hipStream_t stream);

// The same with pos read from device memory (pos_device, one int) and cos /
// sin the whole position tables [s_max][d/2]: one launch shape for every
// position, so a captured graph serves each token.  The grid holds the most
// chunks max_seq_len can need; a pos outside [0, s_max) changes nothing.
hipError_t launch_decode_attention_at(const void* qkv, int n_q, int n_kv, const void* q_norm_w, const void* k_norm_w,
                                      float eps, const void* cos_table, const void* sin_table, void* k_cache,
                                      void* v_cache, int s_max, const int* pos_device, float scale, void* out,
                                      void* workspace, size_t ws_bytes, hipStream_t stream);

// Number of scoring workgroups (= argmax partials per row) the lm_head
// kernel uses for V vocab rows (V % 16 == 0): with NB = V / 16 row-blocks,
// NB if NB <= 512, else (NB - T) / 2 + T with T = 512 + (NB - 512) % 2 (pairs
// of row-blocks, then T single ones).
int lm_head_partials(int V);

// The lm_head workspace: a status header (word 0 counts second stages that
// gave up waiting for a partial) followed by M * lm_head_partials(V) 64-bit
// partials.  It must be zero when first used; every call leaves the partials
// zero again.
constexpr size_t kLmHeadStatusBytes = 64;
inline size_t lm_head_workspace_bytes(int M, int V) {
  return kLmHeadStatusBytes + (size_t)M * (size_t)lm_head_partials(V) * sizeof(ArgmaxPartial);
}

hipError_t launch_lm_head_argmax(const void* w, int V, int K, const void* x, int M, int ldx,
                                 float* logits, int logits_bf16, long long* out_idx,
                                 void* workspace, const void* norm_w, float eps, hipStream_t stream);

// The skinny kernel's plan: `rows` weight rows per workgroup (16, or 32 for a
// gate/up pair), `groups` = N / rows, each K range split over S workgroups
// (S > 1 only with a workspace of `bytes` bytes), for a device of `cus` CUs.
struct SkinnyPlan {
  int rows, groups, S;
  size_t bytes;
};
int skinny_groups(int M);
hipError_t current_device_cus(int* cus_out);
bool skinny_route(int M, int N, int K);
SkinnyPlan skinny_plan(int M, int N, int K, bool silu, int cus, bool has_workspace);
// y = epilogue(x . W^T) for kDecodeMaxM < M <= kSkinnyMaxM (N % 16 == 0, or
// N % 32 == 0 for SiLU*up; K % 32 == 0).  `workspace` (NULL: no split) must
// hold skinny_plan(...).bytes bytes, flags zero (every call leaves them zero).
hipError_t launch_skinny_linear(const void* w, int N, int K, const void* x, int M, int ldx, void* y, int ldy,
                                Epilogue epi, const void* residual, int ldr, void* workspace, size_t ws_bytes,
                                int cus, hipStream_t stream);

// The step-streaming probe (probe.hip, lsk_probe_stream_step): segment s has
// per_cu[s] 1 KB tiles per workgroup starting at tile first[s] + g * per_cu[s].
constexpr int kProbeComputeWaves = 12;
constexpr int kProbeMaxSegments = 256;
struct ProbeSegments {
  int count;
  int per_cu[kProbeMaxSegments];
  unsigned long long first[kProbeMaxSegments];
};
// Workspace words: error, exit counter, checksum sink, the global arrival
// word, 8 group words (16 apart), one flat arrival word per segment, 8 go
// words per segment, then 8 replicas of one tag word per workgroup (mode 3,
// at most kProbeMaxTagGroups workgroups).
constexpr int kProbeWsError = 0;
constexpr int kProbeWsExit = 1;
constexpr int kProbeWsSink = 2;
constexpr int kProbeWsGlobal = 16;
constexpr int kProbeWsGroups = 64;
constexpr int kProbeWsFlat = 256;
constexpr int kProbeWsGo = kProbeWsFlat + kProbeMaxSegments;
constexpr int kProbeMaxTagGroups = 256;
constexpr int kProbeWsTags = kProbeWsGo + 8 * kProbeMaxSegments;
constexpr size_t kProbeWsBytes = (size_t)(kProbeWsTags + 8 * kProbeMaxTagGroups) * 4;
hipError_t launch_probe_step(const void* weights, const ProbeSegments& seg, int mode, int ring, int grid,
                             void* workspace, hipStream_t stream);
hipError_t launch_probe_mfma(int workgroups, int iterations, void* sink, hipStream_t stream);

// Records a HIP failure for lsk_last_error (defined in abi.cpp).
int fail_hip_call(hipError_t err, const char* what);

// The next start/stop event pair of a dispatch timing active on this host
// thread (lsk_dispatch_timing_begin), or false when none is active or its
// pairs are used up (defined in abi.cpp).
bool dispatch_timing_events(hipEvent_t* start, hipEvent_t* stop);

// Every kernel the library launches goes through here: with a dispatch
// timing active, the event pair is bound to the dispatch itself
// (hipExtLaunchKernelGGL), so its elapsed time is the kernel's own duration.
template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                          Args... args) {
  static_assert(sizeof...(KArgs) == sizeof...(Args), "one argument per kernel parameter");
  hipEvent_t start, stop;
  if (dispatch_timing_events(&start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)lds, stream, start, stop, 0u,
                          static_cast<KArgs>(args)...);
  else
    kernel<<<grid, block, lds, stream>>>(static_cast<KArgs>(args)...);
}

// Workspace bytes the split-K prefill path needs on `device` for this shape
// (0 when the shape does not take it).  Sets *status to a HIP error if the
// device query fails.
size_t gemm_workspace_bytes(int device, int M, int N, int K, hipError_t* status);

// Polls of a split-K arrival word before the wait gives up (default
// kSkSpinLimit); applies to launches made after the call.
void set_linear_wait_limit(unsigned polls);

// Prefill GEMM launch (any M >= 1; used for M > kDecodeMaxM).  With a
// workspace (the caller has checked it holds gemm_workspace_bytes()) the
// last partial round of output blocks is split along K over the idle CUs;
// with none, one workgroup per output block.
hipError_t launch_gemm_linear(const void* w, int N, int K, const void* x, int M, int ldx,
                              void* y, int ldy, Epilogue epi, const void* residual, int ldr,
                              void* workspace, size_t ws_bytes, hipStream_t stream);
// The prefill GEMM's plan for M rows of an [N, K] weight on the current
// device, with a workspace (ws_bytes > 0, checked as for the launch) or
// without: {block rows, blocks, split blocks, chunks per split block};
// {0, 0, 0, 1} when the shape takes another kernel.
hipError_t plan_gemm_linear(int M, int N, int K, size_t ws_bytes, int plan[4]);

}  // namespace lsk
