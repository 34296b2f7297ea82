// Host-side driver for the sanitizer build of librq (AddressSanitizer +
// UndefinedBehaviorSanitizer on the host code of api.hip). It calls every entry
// point along the paths that need no GPU: argument validation, handle checks on
// NULL / unknown / dangling handles, the thread-local error message, the status
// strings and the pure helpers. Exit status 0 and no sanitizer report is a pass.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../include/rq.h"

static int failures = 0;
#define EXPECT(cond)                                                   \
  do {                                                                 \
    if (!(cond)) {                                                     \
      std::fprintf(stderr, "EXPECT failed line %d: %s\n", __LINE__, #cond); \
      failures++;                                                      \
    }                                                                  \
  } while (0)

int main() {
  EXPECT(rq_version() == RQ_VERSION);
  for (int s = -2; s <= 9; s++) EXPECT(rq_status_string(s) != nullptr && std::strlen(rq_status_string(s)) > 0);

  int64_t inp = 0;
  EXPECT(rq_nextpad(1, &inp) == RQ_OK && inp == 256);
  EXPECT(rq_nextpad(257, &inp) == RQ_OK && inp == 512);
  EXPECT(rq_nextpad(640, &inp) == RQ_OK && inp == 768);
  EXPECT(rq_nextpad(((int64_t)1 << 40), &inp) == RQ_OK);
  EXPECT(rq_nextpad(0, &inp) == RQ_ERR_SHAPE);
  EXPECT(rq_nextpad(-5, &inp) == RQ_ERR_SHAPE);
  EXPECT(rq_nextpad(INT64_MAX, &inp) == RQ_ERR_SHAPE);
  EXPECT(rq_nextpad(5, nullptr) == RQ_ERR_NULL);
  EXPECT(std::strlen(rq_last_error()) > 0);

  // no GPU here: creating a context fails with a status, never crashes
  rq_ctx ctx = nullptr;
  const int cs = rq_ctx_create(0, &ctx);
  EXPECT(cs != RQ_OK || ctx != nullptr);
  if (cs == RQ_OK) rq_ctx_destroy(ctx);
  EXPECT(rq_ctx_create(-1, &ctx) != RQ_OK);
  EXPECT(rq_ctx_create(0, nullptr) == RQ_ERR_NULL);

  // handles: NULL, unknown (never created) and dangling values are reported, not dereferenced
  std::vector<uint8_t> junk(4096, 0xAB);
  rq_ctx bad_ctx = reinterpret_cast<rq_ctx>(junk.data());
  rq_weight bad_w = reinterpret_cast<rq_weight>(junk.data() + 64);
  EXPECT(rq_ctx_destroy(nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_ctx_destroy(bad_ctx) == RQ_ERR_HANDLE);
  EXPECT(rq_weight_destroy(nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_weight_destroy(bad_w) == RQ_ERR_HANDLE);
  int fmt = 0, sdt = 0, cu = 0, ws = 0, clk = 0;
  int64_t out = 0, in = 0;
  size_t bytes = 0;
  EXPECT(rq_weight_info(bad_w, &fmt, &out, &in, &sdt, &bytes) == RQ_ERR_HANDLE);
  EXPECT(rq_ctx_device_info(bad_ctx, &cu, &ws, &clk) == RQ_ERR_HANDLE);
  void* p = nullptr;
  EXPECT(rq_buf_alloc(bad_ctx, 256, &p) == RQ_ERR_HANDLE);
  EXPECT(rq_buf_free(bad_ctx, junk.data()) == RQ_ERR_HANDLE);
  EXPECT(rq_upload(bad_ctx, junk.data(), junk.data(), 16, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_download(bad_ctx, junk.data(), junk.data(), 16, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_sync(bad_ctx, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_stream_create(bad_ctx, &p) == RQ_ERR_HANDLE);
  EXPECT(rq_ctx_set_kernel_timing(bad_ctx, 1) == RQ_ERR_HANDLE);
  double ms = 0;
  int64_t n = 0;
  EXPECT(rq_ctx_kernel_time(bad_ctx, &ms, &n) == RQ_ERR_HANDLE);

  std::vector<int8_t> codes(64 * 64, 1);
  std::vector<float> scales(64 * 2, 0.5f), x(64, 1.0f), y(64, 0.0f);
  rq_weight w = nullptr;
  EXPECT(rq_weight_create_q8(bad_ctx, codes.data(), scales.data(), 64, 64, &w) == RQ_ERR_HANDLE);
  EXPECT(rq_weight_create_q8(nullptr, codes.data(), scales.data(), 64, 64, &w) == RQ_ERR_HANDLE);
  EXPECT(rq_qmatmul(bad_ctx, bad_w, x.data(), RQ_F32, y.data(), RQ_F32, 1, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_qmatmul_noalloc(bad_ctx, bad_w, x.data(), RQ_F32, y.data(), RQ_F32, 1, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_qmatmul_dx(bad_ctx, bad_w, x.data(), y.data(), 1, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_dequant(bad_ctx, bad_w, y.data(), nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_qlinear_q8(bad_ctx, x.data(), codes.data(), scales.data(), 1, 64, 64, y.data()) == RQ_ERR_HANDLE);
  EXPECT(rq_qlinear_q8_dx(bad_ctx, x.data(), codes.data(), scales.data(), 1, 64, 64, y.data()) == RQ_ERR_HANDLE);
  EXPECT(rq_decode_attention(bad_ctx, x.data(), x.data(), x.data(), y.data(), y.data(), 0, 1, 1, 64, 1e4, 0.125,
                             y.data(), nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_stream_read(bad_ctx, junk.data(), 16, 1, nullptr, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_sgemm(bad_ctx, x.data(), x.data(), y.data(), 2, 2, 2, 1.0f, 0.0f, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_sgemm_tn(bad_ctx, x.data(), x.data(), y.data(), 2, 2, 2, 1.0f, 0.0f, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_sgemm_nt(nullptr, x.data(), x.data(), y.data(), 0, 0, 0, 1.0f, 0.0f, nullptr) == RQ_ERR_HANDLE);
  EXPECT(rq_linear(bad_ctx, x.data(), x.data(), x.data(), y.data(), 2, 2, 2, nullptr) == RQ_ERR_HANDLE);

  // the error message is per thread: a failure in one thread leaves another's message alone
  EXPECT(rq_ctx_destroy(nullptr) == RQ_ERR_HANDLE);
  const std::string mine = rq_last_error();
  std::vector<std::thread> ts;
  for (int t = 0; t < 8; t++)
    ts.emplace_back([] {
      int64_t v;
      for (int i = 0; i < 200; i++) {
        (void)rq_nextpad(-i - 1, &v);
        (void)rq_weight_destroy(nullptr);
        (void)std::strlen(rq_last_error());
      }
    });
  for (auto& t : ts) t.join();
  EXPECT(mine == rq_last_error());

  if (failures) std::fprintf(stderr, "%d expectation(s) failed\n", failures);
  else std::printf("sanitizer driver: all checks passed\n");
  return failures ? 1 : 0;
}
