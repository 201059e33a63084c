// Host-side bounds check of kernel index maps (compiled with g++ by
// tests/test_bounds.py; no GPU).  Every work item of a launch is walked
// through the same index functions the kernels use (csrc/sbq_index.h) and
// each range it reads or writes is checked against the buffer it addresses.
// Prints "ok" or the first violation and exits non-zero.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "sbq_index.h"

using namespace sbq;

static int fail(const char* what, long long a, long long b, long long c, long long d) {
  std::printf("violation: %s (%lld %lld %lld %lld)\n", what, a, b, c, d);
  return 1;
}

// quantize_act_kernel, vector path: x [M, K] with row stride ldx, K % 16 == 0.
// Every 16-value load must lie inside the rows of x: [m * ldx, m * ldx + K).
static int check_act_chunks(int M, int K, long long ldx, bool unclamped) {
  const int Kp = (K + 63) / 64 * 64, cpr = Kp / 16;
  const long long nch = (long long)M * cpr;
  for (long long c = 0; c < nch; ++c) {
    long long src = act_chunk_src(c, cpr, K, ldx);
    if (unclamped) src = (c / cpr) * ldx + (c % cpr) * 16;  // the form without the clamp
    const long long m = src / ldx, k = src - m * ldx;
    if (src < 0 || m >= M || k + 16 > K) return fail("act chunk leaves its row", M, K, c, src);
  }
  return 0;
}

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  if (!std::strcmp(argv[1], "act") && argc == 5)
    return check_act_chunks(std::atoi(argv[2]), std::atoi(argv[3]), std::atoll(argv[4]), false) ? 1
                                                                                                  : (std::puts("ok"), 0);
  if (!std::strcmp(argv[1], "act-unclamped") && argc == 5)
    return check_act_chunks(std::atoi(argv[2]), std::atoi(argv[3]), std::atoll(argv[4]), true) ? 1
                                                                                                : (std::puts("ok"), 0);
  return 2;
}
