// Host-side checks of kernel index arithmetic (compiled with g++ by
// tests/test_bounds.py; no GPU), through the same functions the kernels use
// (csrc/sbq_index.h):
//   * bounds: every work item of a launch is walked through an index map and
//     each range it reads or writes is checked against the buffer it
//     addresses (prints "ok" or the first violation and exits non-zero);
//   * the fused greedy token's key order: the index with the largest key over
//     values read from stdin.
#include <cmath>
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

// Fused greedy token: the index whose argmax_key is largest over the values
// read from stdin (one per line).  `fold_zero` false plants the mistake of
// ordering -0 below +0.
static int pick_argmax(bool fold_zero) {
  unsigned long long best = 0;
  float v;
  int n = 0;
  while (std::scanf("%f", &v) == 1) {
    unsigned long long k = argmax_key(v, n);
    if (!fold_zero && v == 0.0f && std::signbit(v)) k = ((unsigned long long)0x7fffffffu << 32) | (k & 0xffffffffu);
    if (k > best) best = k;
    ++n;
  }
  std::printf("%d\n", best ? argmax_key_index(best) : -1);
  return 0;
}

// The fused argmax's slot arithmetic against brute-force counting: every
// slot's member count, the occupied slots, and that the members of all slots
// add up to the grid.
static int check_argmax_slots() {
  const unsigned slots = 64;
  for (unsigned nblk = 1; nblk <= 5000; ++nblk) {
    unsigned members[64] = {0}, total = 0, used = 0;
    for (unsigned b = 0; b < nblk; ++b) ++members[b % slots];
    for (unsigned s = 0; s < slots; ++s) {
      if (argmax_slot_members(nblk, s, slots) != members[s]) return fail("slot members", nblk, s, members[s], 0);
      total += members[s];
      used += members[s] > 0;
    }
    if (total != nblk || argmax_slots_used(nblk, slots) != used) return fail("slots used", nblk, used, total, 0);
  }
  std::puts("ok");
  return 0;
}

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  if (!std::strcmp(argv[1], "argmax")) return pick_argmax(true);
  if (!std::strcmp(argv[1], "argmax-slots")) return check_argmax_slots();
  if (!std::strcmp(argv[1], "argmax-unfolded-zero")) return pick_argmax(false);
  if (!std::strcmp(argv[1], "act") && argc == 5)
    return check_act_chunks(std::atoi(argv[2]), std::atoi(argv[3]), std::atoll(argv[4]), false) ? 1
                                                                                                  : (std::puts("ok"), 0);
  if (!std::strcmp(argv[1], "act-unclamped") && argc == 5)
    return check_act_chunks(std::atoi(argv[2]), std::atoi(argv[3]), std::atoll(argv[4]), true) ? 1
                                                                                                : (std::puts("ok"), 0);
  return 2;
}
