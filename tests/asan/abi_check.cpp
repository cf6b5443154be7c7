// Drives the product library's host code under AddressSanitizer: geometry validation over random
// and adversarial geometries, workspace sizes and layouts (monotone, aligned, matching the
// size queries, int and int64 forms), error strings, argument validation of every entry point,
// the no-allocation entry point's size check. Every call here returns before any HIP call, so it
// runs without a GPU.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "justgoal_moe.h"

#define CHECK(c)                                                          \
  do {                                                                    \
    if (!(c)) {                                                           \
      std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
      return 1;                                                           \
    }                                                                     \
  } while (0)

int main() {
  std::mt19937 rng(7);
  auto pick = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
  int valid = 0, invalid = 0;
  for (int it = 0; it < 20000; ++it) {
    moe_geometry g;
    g.hidden = 128 * pick(-1, 130) + (pick(0, 9) == 0 ? pick(1, 127) : 0);
    g.intermediate = 128 * pick(-1, 130);
    g.num_experts = 64 * pick(-1, 9);
    g.local_experts = pick(-2, 300);
    g.top_k = pick(-1, 10);
    g.n_group = pick(0, 20);
    g.topk_group = pick(0, 20);
    g.routing_method = pick(-1, 2);
    const int T = pick(-3, 70000);
    int64_t off[MOE_WS_NUM_REGIONS + 1];
    std::memset(off, 0xff, sizeof off);
    const int rc = moe_workspace_layout(&g, T, off);
    const int64_t n = moe_workspace_bytes_ex(&g, T);
    if (rc == MOE_OK) {
      ++valid;
      CHECK(T >= 0);
      CHECK(n == off[MOE_WS_NUM_REGIONS]);
      for (int i = 0; i < MOE_WS_NUM_REGIONS; ++i) CHECK(off[i] <= off[i + 1] && off[i] % 256 == 0);
      const int64_t kl = g.top_k < g.local_experts ? g.top_k : g.local_experts;
      CHECK(off[MOE_WS_PARTIAL] - off[MOE_WS_C] >= (int64_t)T * kl * g.intermediate * 2);
      CHECK(off[MOE_WS_CHUNK_COUNTS] - off[MOE_WS_PARTIAL] >= (int64_t)T * (kl - 1) * g.hidden * 2);
    } else {
      ++invalid;
      CHECK(rc < 0 && n < 0);
      CHECK(std::strlen(moe_error_string(rc)) > 0);
    }
    // argument validation that must fail before any device work
    char dummy[16];
    void* p = dummy;
    CHECK(moe_run_ex(&g, nullptr, nullptr, p, p, p, p, p, p, 0, 1.0f, p, p, T > 0 ? T : 1,
                     nullptr) != MOE_OK);
    CHECK(moe_run_ex(&g, p, p, p, p, p, p, p, p, 0, 1.0f, p, p, -1 - (T & 7), nullptr) != MOE_OK);
    CHECK(moe_route_ex(&g, p, p, 0, 1.0f, p, -1, nullptr) != MOE_OK);
  }
  CHECK(valid > 500 && invalid > 500);
  CHECK(moe_workspace_layout(nullptr, 1, nullptr) == MOE_ERR_INVALID_ARG);
  // the reference's int size query: exact up to 16107 DS-V3 tokens, an error code beyond
  const moe_geometry ds = {7168, 2048, 256, 32, 8, 8, 4, MOE_ROUTING_DS};
  for (int T = 0; T <= 20000; T += 37) {
    const int n = moe_workspace_bytes(T);
    const int64_t n64 = moe_workspace_bytes_ex(&ds, T);
    if (n64 <= INT32_MAX) CHECK(n == n64);
    else CHECK(n == MOE_ERR_INVALID_ARG);
  }
  CHECK(moe_workspace_bytes(-5) < 0);
  // tokens beyond the ABI limit, and the no-allocation entry point's size check
  char dummy[16];
  void* p = dummy;
  CHECK(moe_run(p, p, p, p, p, p, p, p, 0, 2.5f, p, p, 65536, nullptr) == MOE_ERR_INVALID_ARG);
  CHECK(moe_run_noalloc(&ds, p, p, p, p, p, p, p, p, 0, 2.5f, p, 504, nullptr) ==
        MOE_ERR_SCRATCH_SIZE);
  CHECK(moe_run_noalloc(&ds, p, p, p, p, p, p, p, p, 0, 2.5f, p, -1, nullptr) ==
        MOE_ERR_INVALID_ARG);
  // stage events: wrong counts and null entries are refused; 0 turns timing off
  void* ev[MOE_NUM_STAGES + 1] = {};
  CHECK(moe_set_stage_events(ev, 3) == MOE_ERR_INVALID_ARG);
  CHECK(moe_set_stage_events(ev, MOE_NUM_STAGES + 1) == MOE_ERR_INVALID_ARG);
  CHECK(moe_set_stage_events(nullptr, MOE_NUM_STAGES + 1) == MOE_ERR_INVALID_ARG);
  CHECK(moe_set_stage_events(nullptr, 0) == MOE_OK);
  CHECK(moe_quantize_activations(p, 4, 100, p, p, nullptr) == MOE_ERR_INVALID_ARG);
  CHECK(moe_quantize_activations(nullptr, 4, 128, p, p, nullptr) == MOE_ERR_INVALID_ARG);
  for (int rc = -6; rc <= 3; ++rc) CHECK(moe_error_string(rc) != nullptr);
  std::printf("abi_check: %d valid and %d invalid random geometries: ok\n", valid, invalid);
  return 0;
}
