// Compares hi_amd/csrc/exact_expf.h (host build) with the host glibc expf:
// every float in [-104, 0] plus every 61st bit pattern elsewhere.
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <string.h>

#include "exact_expf.h"

namespace {
const int kThreads = 8;
long long g_bad[kThreads];
long long g_count[kThreads];

void* work(void* arg) {
  const long id = (long)arg;
  // negatives down to -104 (bits 0x80000000 .. 0xC2D00000), exhaustively
  for (uint64_t b = 0x80000000ull + id; b <= 0xC2D00000ull; b += kThreads) {
    uint32_t u = (uint32_t)b;
    float x;
    memcpy(&x, &u, 4);
    float a = hi_rocm::exact_expf(x), r = expf(x);
    g_bad[id] += memcmp(&a, &r, 4) != 0;
    g_count[id]++;
  }
  // everything else, sampled
  for (uint64_t b = (uint64_t)id * 61; b <= 0xFFFFFFFFull; b += 61 * kThreads) {
    if (b >= 0x80000000ull && b <= 0xC2D00000ull) continue;
    uint32_t u = (uint32_t)b;
    float x;
    memcpy(&x, &u, 4);
    float a = hi_rocm::exact_expf(x), r = expf(x);
    if (isnan(r) && isnan(a)) { g_count[id]++; continue; }
    g_bad[id] += memcmp(&a, &r, 4) != 0;
    g_count[id]++;
  }
  return nullptr;
}
}  // namespace

int main() {
  pthread_t th[kThreads];
  for (long i = 0; i < kThreads; ++i) pthread_create(&th[i], nullptr, work, (void*)i);
  long long bad = 0, cnt = 0;
  for (int i = 0; i < kThreads; ++i) {
    pthread_join(th[i], nullptr);
    bad += g_bad[i];
    cnt += g_count[i];
  }
  printf("checked %lld inputs, mismatches %lld\n", cnt, bad);
  return bad == 0 ? 0 : 1;
}
