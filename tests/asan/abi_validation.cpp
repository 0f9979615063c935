// Host-only driver for the sanitizer build of the C ABI's argument validation
// (csrc/wq_abi.hip, csrc/abi.hip), run by tests/test_asan_abi.py on the CPU.
//
// Every call passes arguments that the validation must reject (or accept as an empty
// problem) before any kernel launch: the launchers below stand in for the kernel files
// and abort if a call reaches them. Built with AddressSanitizer and
// UndefinedBehaviorSanitizer on the host code (no recovery), so an out-of-bounds access,
// a signed overflow or a misaligned load anywhere on these paths ends the run.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "wq.h"

namespace mls {
namespace {
[[noreturn]] void reached(const char* what) {
  std::fprintf(stderr, "validation let a call through to %s\n", what);
  std::abort();
}
}  // namespace
int launch_gemv_wq(int, const WqArgs&) { reached("launch_gemv_wq"); }
int launch_gemv_rows(int, const WqArgs&) { reached("launch_gemv_rows"); }
int launch_gemv_mfma(int, const WqArgs&) { reached("launch_gemv_mfma"); }
int launch_gemv_mfma_f32(int, const WqArgs&) { reached("launch_gemv_mfma_f32"); }
int launch_gemm_small(int, const WqArgs&) { reached("launch_gemm_small"); }
int launch_gemm_wq_mfma(int, const WqArgs&) { reached("launch_gemm_wq_mfma"); }
int launch_gemm_wq_generic(int, const WqArgs&) { reached("launch_gemm_wq_generic"); }
int launch_grouped_int4(const GroupedArgs&) { reached("launch_grouped_int4"); }
int launch_grouped_gate_up(const GroupedArgs&, const uint8_t*, const void*) { reached("launch_grouped_gate_up"); }
int launch_grouped_int4_partial(const GroupedArgs&, int, float*, int64_t, int64_t) {
  reached("launch_grouped_int4_partial");
}
int grouped_splits(int64_t, int, int64_t, int64_t, int) { return 1; }
int launch_gemm_small_split(int, const WqArgs&, int64_t) { reached("launch_gemm_small_split"); }
int launch_gemm_wq_mfma_split(int, const WqArgs&, int64_t) { reached("launch_gemm_wq_mfma_split"); }
int launch_gemv_mfma_split(int, const WqArgs&) { reached("launch_gemv_mfma_split"); }
int launch_split_rows(const float*, int64_t, int64_t, int64_t, void*, hipStream_t) { reached("launch_split_rows"); }
}  // namespace mls

namespace {

int failures = 0;

void expect(const char* what, int rc, int want, const char* msg_part = nullptr) {
  const char* msg = mls_last_error();
  const bool ok = rc == want && (msg_part == nullptr || std::strstr(msg, msg_part) != nullptr);
  if (!ok) {
    std::fprintf(stderr, "FAIL %s: rc=%d (want %d), last error \"%s\"\n", what, rc, want, msg);
    ++failures;
  }
}

// distinct non-null addresses that are never dereferenced
const void* P(int i) { return reinterpret_cast<const void*>(static_cast<uintptr_t>(0x1000 * (i + 1))); }
template <typename T>
const T* PT(int i) { return static_cast<const T*>(P(i)); }

constexpr int BF = MLS_BF16, F16 = MLS_F16, F32 = MLS_F32;
constexpr int64_t BIG = int64_t(1) << 40;

void int8_gemm_cases() {
  auto call = [](const void* a, int adt, int64_t lda, const void* w, int64_t ldw, const void* s, int sdt, void* c,
                 int cdt, int64_t ldc, int64_t M, int64_t N, int64_t K) {
    return mls_int8_gemm(a, adt, lda, static_cast<const int8_t*>(w), ldw, s, sdt, c, cdt, ldc, M, N, K, nullptr);
  };
  void* c = const_cast<void*>(P(3));
  expect("int8 negative M", call(P(0), BF, 64, P(1), 64, P(2), F32, c, BF, 32, -1, 32, 64), MLS_ERR_ARG, "negative");
  expect("int8 negative K", call(P(0), BF, 64, P(1), 64, P(2), F32, c, BF, 32, 4, 32, INT64_MIN), MLS_ERR_ARG);
  expect("int8 bad dtype", call(P(0), 7, 64, P(1), 64, P(2), F32, c, 7, 32, 4, 32, 64), MLS_ERR_ARG, "dtype");
  expect("int8 out dtype", call(P(0), BF, 64, P(1), 64, P(2), F32, c, F16, 32, 4, 32, 64), MLS_ERR_ARG);
  expect("int8 scale dtype", call(P(0), BF, 64, P(1), 64, P(2), BF, c, BF, 32, 4, 32, 64), MLS_ERR_ARG, "scale");
  expect("int8 null a", call(nullptr, BF, 64, P(1), 64, P(2), F32, c, BF, 32, 4, 32, 64), MLS_ERR_ARG, "null");
  expect("int8 null c", call(P(0), BF, 64, P(1), 64, P(2), F32, nullptr, BF, 32, 4, 32, 64), MLS_ERR_ARG, "null");
  expect("int8 lda < K", call(P(0), BF, 63, P(1), 64, P(2), F32, c, BF, 32, 4, 32, 64), MLS_ERR_ARG, "leading");
  expect("int8 ldc < N", call(P(0), BF, 64, P(1), 64, P(2), F32, c, BF, 31, 4, 32, 64), MLS_ERR_ARG, "leading");
  expect("int8 empty M", call(nullptr, BF, 64, nullptr, 64, nullptr, F32, nullptr, BF, 32, 0, 32, 64), MLS_OK);
  expect("int8 empty N", call(nullptr, BF, 64, nullptr, 64, nullptr, F32, nullptr, BF, 32, 4, 0, 64), MLS_OK);
  // sizes whose products overflow 64 bits must be rejected without overflowing
  expect("int8 huge M N", call(P(0), BF, BIG, P(1), BIG, P(2), F32, c, BF, BIG, BIG, BIG, BIG), MLS_ERR_UNSUPPORTED,
         "too large");
  expect("int8 max M N", call(P(0), BF, INT64_MAX, P(1), INT64_MAX, P(2), F32, c, BF, INT64_MAX, INT64_MAX,
                              INT64_MAX, 64),
         MLS_ERR_UNSUPPORTED, "too large");
}

void int4_gemm_cases() {
  auto call = [](int64_t ld_sn, int64_t ld_sg, int group, int64_t M, int64_t N, int64_t K, int64_t ldw = 32) {
    return mls_int4_gemm(P(0), BF, 64, PT<uint8_t>(1), ldw, P(2), F16, ld_sn, ld_sg, group,
                         const_cast<void*>(P(3)), BF, 64, M, N, K, nullptr);
  };
  expect("int4 group 0", call(2, 1, 0, 4, 64, 64), MLS_ERR_ARG, "group");
  expect("int4 group negative", call(2, 1, -32, 4, 64, 64), MLS_ERR_ARG, "group");
  expect("int4 K not multiple of group", call(2, 1, 48, 4, 64, 64), MLS_ERR_ARG, "multiple");
  expect("int4 odd K", call(2, 1, 1, 4, 64, 63), MLS_ERR_ARG);
  expect("int4 negative scale stride", call(-2, 1, 32, 4, 64, 64), MLS_ERR_ARG, "stride");
  expect("int4 ldw < K/2", call(2, 1, 32, 4, 64, 64, 31), MLS_ERR_ARG, "leading");
  expect("int4 huge", call(2, 1, 32, BIG, BIG, 64), MLS_ERR_ARG);
}

void workspace_cases() {
  // fp32 activations with M > 16 take the split route: the workspace is checked first
  void* c = const_cast<void*>(P(3));
  const int64_t need = mls_wq_gemm_workspace(8, 64, 32, 64, F32, 0);
  if (need != 128 * 64 * 2) {
    std::fprintf(stderr, "FAIL workspace size %lld\n", (long long)need);
    ++failures;
  }
  auto w8 = [&](void* ws, int64_t bytes, int64_t M) {
    return mls_int8_gemm_ws(P(0), F32, 64, PT<int8_t>(1), 64, P(2), F32, c, F32, 32, M, 32, 64, ws, bytes, nullptr);
  };
  void* ws = const_cast<void*>(P(15));  // 0x10000: 256-byte aligned
  expect("int8 ws null", w8(nullptr, need, 64), MLS_ERR_ARG, "workspace");
  expect("int8 ws short", w8(ws, need - 1, 64), MLS_ERR_ARG, "workspace");
  expect("int8 ws misaligned", w8(static_cast<char*>(ws) + 16, need, 64), MLS_ERR_ARG, "aligned");
  expect("int8 ws negative M", w8(ws, need, -1), MLS_ERR_ARG, "negative");
  expect("int8 ws empty M", w8(nullptr, 0, 0), MLS_OK);
  expect("int8 ws huge", mls_int8_gemm_ws(P(0), F32, BIG, PT<int8_t>(1), BIG, P(2), F32, c, F32, BIG, BIG, BIG, BIG,
                                          ws, need, nullptr),
         MLS_ERR_UNSUPPORTED, "too large");
  expect("int4 ws null", mls_int4_gemm_ws(P(0), F32, 64, PT<uint8_t>(1), 32, P(2), F16, 1, 1, 64, c, F32, 32, 64, 32,
                                          64, nullptr, 0, nullptr),
         MLS_ERR_ARG, "workspace");
  expect("int4 ws group", mls_int4_gemm_ws(P(0), F32, 64, PT<uint8_t>(1), 32, P(2), F16, 1, 1, 48, c, F32, 32, 64, 32,
                                           64, ws, need, nullptr),
         MLS_ERR_ARG, "group");
  if (mls_wq_gemm_workspace(8, 1, 32, 64, F32, 0) != 0 || mls_wq_gemm_workspace(4, 64, 32, 64, F32, 32) != 0 ||
      mls_wq_gemm_workspace(8, 64, 32, 64, BF, 0) != 0 || mls_wq_gemm_workspace(8, INT64_MAX, 32, 64, F32, 0) != 0) {
    std::fprintf(stderr, "FAIL workspace query outside the split route\n");
    ++failures;
  }
}

void grouped_cases() {
  const int32_t* off = PT<int32_t>(4);
  const int32_t* rows = PT<int32_t>(5);
  void* c = const_cast<void*>(P(3));
  auto g = [&](int E, int64_t M, int64_t K, int64_t west, int64_t sest, const int32_t* seg) {
    return mls_int4_grouped_gemm(P(0), BF, 64, seg, E, M, PT<uint8_t>(1), west, 32, P(2), F16, sest, 2, 1, 32, c,
                                 BF, 64, 64, K, nullptr);
  };
  expect("grouped E=0", g(0, 16, 64, 1024, 128, off), MLS_ERR_ARG, "E=0");
  expect("grouped K=0", g(2, 16, 0, 1024, 128, off), MLS_ERR_ARG, "K=0");
  expect("grouped negative stride", g(2, 16, 64, -1, 128, off), MLS_ERR_ARG, "stride");
  expect("grouped null offsets", g(2, 16, 64, 1024, 128, nullptr), MLS_ERR_ARG, "seg_off");
  expect("grouped empty", g(2, 0, 64, 1024, 128, nullptr), MLS_OK);
  expect("grouped fp32 activations",
         mls_int4_grouped_gemm(P(0), F32, 64, off, 2, 16, PT<uint8_t>(1), 1024, 32, P(2), F16, 128, 2, 1, 32, c, F32,
                               64, 64, 64, nullptr),
         MLS_ERR_UNSUPPORTED);
  auto gr = [&](const int32_t* r, int64_t src) {
    return mls_int4_grouped_gemm_rows(P(0), BF, 64, r, src, off, 2, 16, PT<uint8_t>(1), 1024, 32, P(2), F16, 128,
                                      2, 1, 32, c, BF, 64, 64, 64, nullptr);
  };
  expect("grouped rows null index", gr(nullptr, 8), MLS_ERR_ARG, "a_rows");
  expect("grouped rows no source rows", gr(rows, 0), MLS_ERR_ARG, "a_src_rows");
  auto gu = [&](const uint8_t* wu, const void* su, int64_t K) {
    return mls_int4_grouped_gate_up(P(0), BF, 64, off, 2, 16, PT<uint8_t>(1), wu, 1024, 32, P(2), su, F16, 128, 2,
                                    1, 32, c, BF, 64, 64, K, nullptr);
  };
  expect("gate/up null up", gu(nullptr, P(6), 64), MLS_ERR_ARG, "null");
  expect("gate/up null up scales", gu(PT<uint8_t>(7), nullptr, 64), MLS_ERR_ARG, "null");
  expect("gate/up K=0", gu(PT<uint8_t>(7), P(6), 0), MLS_ERR_ARG, "K=0");
  expect("gate/up rows null index",
         mls_int4_grouped_gate_up_rows(P(0), BF, 64, nullptr, 8, off, 2, 16, PT<uint8_t>(1), PT<uint8_t>(7), 1024,
                                       32, P(2), P(6), F16, 128, 2, 1, 32, c, BF, 64, 64, 64, nullptr),
         MLS_ERR_ARG, "a_rows");
  float* part = static_cast<float*>(const_cast<void*>(P(8)));
  auto gp = [&](int splits, int64_t sstride, int64_t K) {
    return mls_int4_grouped_gemm_partial(P(0), BF, 64, off, 2, 16, PT<uint8_t>(1), 1024, 32, P(2), F16, 128, 2, 1,
                                         32, splits, part, 64, sstride, 64, K, nullptr);
  };
  expect("partial splits 0", gp(0, 16 * 64, 64), MLS_ERR_ARG, "splits");
  expect("partial splits 65", gp(65, 16 * 64, 64), MLS_ERR_ARG, "splits");
  expect("partial short split stride", gp(2, 16 * 64 - 1, 64), MLS_ERR_ARG, "stride");
  expect("partial K=0", gp(2, 16 * 64, 0), MLS_ERR_ARG, "K=0");
}

}  // namespace

int main() {
  if (mls_abi_version() != MLS_ABI_VERSION) {
    std::fprintf(stderr, "abi version %d != %d\n", mls_abi_version(), MLS_ABI_VERSION);
    return 1;
  }
  int8_gemm_cases();
  int4_gemm_cases();
  workspace_cases();
  grouped_cases();
  // a long message is truncated, not overrun
  char name[600];
  std::memset(name, 'x', sizeof(name) - 1);
  name[sizeof(name) - 1] = 0;
  mls::fail(MLS_ERR_ARG, "%s", name);
  if (std::strlen(mls_last_error()) >= sizeof(name)) {
    std::fprintf(stderr, "FAIL: last error not truncated\n");
    ++failures;
  }
  if (failures) return 1;
  std::printf("abi validation: all cases passed\n");
  return 0;
}
