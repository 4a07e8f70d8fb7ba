// Drives the host-side rules of the C ABI (leanstack_amd/csrc/host_rules.cpp)
// under AddressSanitizer and UndefinedBehaviorSanitizer: pack / unpack round
// trips on exactly-sized heap buffers (an index past either buffer is reported
// by ASan) and the rejection paths of the argument validators.  Built and run
// by tests/test_host_sanitizers.py with g++; prints "ok" and exits 0 when every
// check holds.

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <random>

#include "leanstack_amd.h"
#include "lsk_host.h"

namespace {

int g_failures = 0;

void expect(bool cond, const char* what) {
  if (!cond) {
    std::printf("FAILED: %s (last error: %s)\n", what, lsk_last_error());
    ++g_failures;
  }
}

void round_trip(int N, int K, int layout, unsigned seed) {
  const size_t n = (size_t)N * K;
  expect(lsk_packed_bytes(layout, N, K) == n * 2, "packed byte count");
  std::unique_ptr<uint16_t[]> w(new uint16_t[n]), packed(new uint16_t[n]), back(new uint16_t[n]);
  std::mt19937 rng(seed);
  for (size_t i = 0; i < n; ++i) w[i] = (uint16_t)rng();
  expect(lsk_pack_bf16(w.get(), N, K, layout, packed.get()) == LSK_OK, "pack");
  std::memset(back.get(), 0xff, n * 2);
  expect(lsk_unpack_bf16(packed.get(), N, K, layout, back.get()) == LSK_OK, "unpack");
  expect(std::memcmp(w.get(), back.get(), n * 2) == 0, "unpack(pack(W)) == W");
  // Packed row 0 of tile (0, 0) for lane 0: W[source row 0][0..7] -- the layout's first 16 bytes.
  expect(std::memcmp(packed.get(), w.get(), 16) == 0, "first lane of the first tile");
}

}  // namespace

int main() {
  round_trip(16, 32, LSK_LAYOUT_MFMA16X32, 1);
  round_trip(48, 96, LSK_LAYOUT_MFMA16X32, 2);
  round_trip(64, 2560, LSK_LAYOUT_MFMA16X32, 3);
  round_trip(32, 64, LSK_LAYOUT_MFMA16X32_GATEUP, 4);
  round_trip(96, 160, LSK_LAYOUT_MFMA16X32_GATEUP, 5);

  uint16_t one[16 * 32] = {};
  uint16_t out[16 * 32];
  expect(lsk_pack_bf16(one, 17, 32, LSK_LAYOUT_MFMA16X32, out) == LSK_ERR_INVALID, "N % 16");
  expect(lsk_pack_bf16(one, 16, 33, LSK_LAYOUT_MFMA16X32, out) == LSK_ERR_INVALID, "K % 32");
  expect(lsk_pack_bf16(one, 16, 32, 9, out) == LSK_ERR_LAYOUT, "unknown layout");
  expect(lsk_pack_bf16(one, 16, 32, LSK_LAYOUT_MFMA16X32_GATEUP, out) == LSK_ERR_INVALID, "gate_up needs pairs");
  expect(lsk_pack_bf16(nullptr, 16, 32, LSK_LAYOUT_MFMA16X32, out) == LSK_ERR_INVALID, "null source");
  expect(lsk_unpack_bf16(one, 16, 32, LSK_LAYOUT_MFMA16X32, nullptr) == LSK_ERR_INVALID, "null destination");
  expect(lsk_packed_bytes(LSK_LAYOUT_MFMA16X32, -16, 32) == 0, "negative N");
  expect(std::strlen(lsk_last_error()) > 0, "a rejection leaves a message");

  // Validators with aligned fake addresses: nothing is dereferenced.
  const void* p = reinterpret_cast<const void*>(uintptr_t(0x10000));
  void* q = reinterpret_cast<void*>(uintptr_t(0x20000));
  using lsk::check_linear_args;
  expect(check_linear_args(p, 1, 6144, 2560, p, 1, 2560, q, 6144, 0, nullptr, 0) == LSK_OK, "valid linear");
  expect(check_linear_args(p, 1, 6144, 2560, p, 0, 2560, q, 6144, 0, nullptr, 0) == LSK_ERR_INVALID, "M = 0");
  expect(check_linear_args(p, 1, 6144, 2560, p, 1, 2552, q, 6144, 0, nullptr, 0) == LSK_ERR_INVALID, "ldx < K");
  expect(check_linear_args(p, 1, 6144, 2560, (const char*)p + 2, 1, 2560, q, 6144, 0, nullptr, 0) == LSK_ERR_INVALID,
         "misaligned x");
  expect(check_linear_args(p, 1, 6144, 2560, p, 1, 2560, q, 6144, 1, nullptr, 0) == LSK_ERR_INVALID,
         "SiLU without the gate_up layout");
  expect(check_linear_args(p, 1, 6144, 2560, p, 1, 2560, q, 6144, 2, nullptr, 0) == LSK_ERR_INVALID,
         "residual add without a residual");
  expect(check_linear_args(p, 2, 19456, 2560, p, 4, 2560, q, 9728, 1, nullptr, 0) == LSK_OK, "valid gate_up");
  expect(lsk::check_attention_args(p, 32, 8, 128, p, p, 1e-6f, p, p, p, p, 4096, 0.088f, q) == LSK_OK,
         "valid attention");
  expect(lsk::check_attention_args(p, 32, 8, 64, p, p, 1e-6f, p, p, p, p, 4096, 0.088f, q) == LSK_ERR_INVALID,
         "head_dim 64");
  expect(lsk::check_attention_args(p, 24, 8, 128, p, p, 1e-6f, p, p, p, p, 4096, 0.088f, q) == LSK_ERR_INVALID,
         "group of 3");
  expect(lsk::check_attention_args(p, 32, 8, 128, p, p, -1.f, p, p, p, p, 4096, 0.088f, q) == LSK_ERR_INVALID,
         "negative eps");
  const long long* idx = reinterpret_cast<const long long*>(uintptr_t(0x30000));
  expect(lsk::check_lm_head(p, 1, 151936, 2560, p, 8, 2560, nullptr, 0, idx) == LSK_OK, "valid lm_head");
  expect(lsk::check_lm_head(p, 2, 151936, 2560, p, 8, 2560, nullptr, 0, idx) == LSK_ERR_LAYOUT, "lm_head layout");
  expect(lsk::check_lm_head(p, 1, 151936, 2560, p, 17, 2560, nullptr, 0, idx) == LSK_ERR_INVALID, "lm_head M = 17");
  expect(lsk::check_lm_head(p, 1, 151928, 2560, p, 1, 2560, nullptr, 0, idx) == LSK_ERR_INVALID, "V % 16");
  expect(lsk::check_lm_head(p, 1, 18992, 2560, p, 1, 2560, nullptr, 0, idx) == LSK_OK, "odd count of row-blocks");

  if (g_failures) {
    std::printf("%d checks failed\n", g_failures);
    return 1;
  }
  std::printf("ok\n");
  return 0;
}
