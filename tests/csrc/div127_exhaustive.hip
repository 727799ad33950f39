// Exhaustive host check of lbk::div127 (lowbit_amd/csrc/lb_device.h), the division by
// 127 of the one-row W4A8 quantizer: for every non-negative finite float32 a (and +inf)
// it must equal the IEEE quotient a / 127.0f bit for bit. Built host-only (no device
// code) with floating-point contraction off, so every operation rounds as written.
// Prints "checked <count> mismatches <count> first <hex>" and exits 0 when none differ.
// With the argument "plain" it checks the uncorrected product fl(a * fl(1/127)) over
// [1, 2) instead: that one differs from the quotient, so the check must find mismatches.
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "lb_device.h"

static float from_bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

static uint32_t to_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

static float plain_product(float a) { return a * (1.0f / 127.0f); }

int main(int argc, char **argv) {
  const bool plain = argc > 1 && std::strcmp(argv[1], "plain") == 0;
  const uint64_t begin = plain ? 0x3F800000ull : 0ull;
  const uint64_t end = plain ? 0x40000000ull : 0x7F800001ull;  // +0 .. +inf inclusive
  unsigned nt = std::thread::hardware_concurrency();
  nt = nt == 0 ? 1 : (nt > 16 ? 16 : nt);
  std::atomic<uint64_t> bad{0};
  std::atomic<uint32_t> first{0xFFFFFFFFu};
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < nt; t++) {
    pool.emplace_back([&, t] {
      // blocks of 2^16 patterns dealt round-robin: the subnormal range, whose
      // arithmetic is slow on x86, is shared by every thread
      const uint64_t blk = 1ull << 16;
      uint64_t nbad = 0;
      uint32_t fb = 0xFFFFFFFFu;
      for (uint64_t lo = begin + t * blk; lo < end; lo += nt * blk) {
        const uint64_t hi = lo + blk < end ? lo + blk : end;
        for (uint64_t u = lo; u < hi; u++) {
          const float a = from_bits((uint32_t)u);
          const float got = plain ? plain_product(a) : lbk::div127(a);
          if (to_bits(got) != to_bits(a / 127.0f)) {
            nbad++;
            if ((uint32_t)u < fb) fb = (uint32_t)u;
          }
        }
      }
      bad += nbad;
      uint32_t cur = first.load();
      while (fb < cur && !first.compare_exchange_weak(cur, fb)) {
      }
    });
  }
  for (auto &th : pool) th.join();
  std::printf("checked %llu mismatches %llu first 0x%08x\n", (unsigned long long)(end - begin),
              (unsigned long long)bad.load(), first.load());
  return bad.load() == 0 ? 0 : 1;
}
