// Checks hi_amd/csrc/exact_fold.h (host build) against a literal sequential
// f32 fold, acc = acc + x left to right, on randomised inputs built to hit
// the hard cases: exact half-ulp terms (both parities), subnormal starts,
// terms above the running sum, long runs of equal terms, sums landing next
// to powers of two, and threshold searches.
//
// Three emulations are checked: the term-by-term integer process (classify
// and compose with one real add per binade crossing), run_walk on runs of
// equal terms, and run_find for the >= and > thresholds.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "exact_fold.h"

using namespace hi_rocm::fold;

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t next_u64() {
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
double unif() { return (double)(next_u64() >> 11) / 9007199254740992.0; }

float seq_fold(float a, const std::vector<float>& x) {
  for (float v : x) a = a + v;
  return a;
}

bool same(float a, float b) { return fbits(a) == fbits(b) || (a == 0.f && b == 0.f); }

// One random non-negative term of a chosen flavour relative to a scale.
float term(int flavour, float scale) {
  switch (flavour) {
    case 0: return (float)(unif() * scale);
    case 1: return (float)(exp(-unif() * 30.0) * scale);                 // wide range
    case 2: return ldexpf((float)(1 + (next_u64() & 7)), -(int)(next_u64() % 40));  // short mantissas: halves
    case 3: return bfloat((uint32_t)(next_u64() % 0x00800000u));         // subnormals
    case 4: return (float)(unif() < 0.5 ? 0.0 : unif() * scale);
    default: return ldexpf(1.0f, -(int)(next_u64() % 150));              // powers of two
  }
}

// The term-by-term integer emulation: maps within the binade, one real add
// at each crossing.
float emulate_terms(float a, const std::vector<float>& x) {
  size_t i = 0;
  while (i < x.size()) {
    const int e = binade(a);
    const uint32_t A = to_A(a);
    Map acc = map_identity();
    size_t j = i;
    for (; j < x.size(); ++j) {
      const Map nx = compose(acc, run_map(classify(x[j], e), 1u));
      if ((uint64_t)A + apply(nx, A & 1u) >= kTop) break;
      acc = nx;
    }
    a = from_A(A + apply(acc, A & 1u), e);
    if (j < x.size()) a = a + x[j];  // the crossing term, as a real add
    i = j + 1;
  }
  return a;
}

long long g_bad = 0, g_cases = 0;
void expect(bool ok, const char* what, int trial) {
  ++g_cases;
  if (!ok) {
    if (g_bad < 20) printf("mismatch: %s (trial %d)\n", what, trial);
    ++g_bad;
  }
}

}  // namespace

int main() {
  // 1. sequences of single terms
  for (int trial = 0; trial < 20000; ++trial) {
    const int n = 1 + (int)(next_u64() % 400);
    const int flav = (int)(next_u64() % 6);
    const float scale = ldexpf(1.0f, (int)(next_u64() % 20) - 10);
    std::vector<float> x(n);
    for (int i = 0; i < n; ++i) x[i] = term((i % 7 == 0) ? (int)(next_u64() % 6) : flav, scale);
    float a0 = 0.f;
    switch (trial % 5) {
      case 0: a0 = -0.0f; break;
      case 1: a0 = 0.f; break;
      case 2: a0 = term(3, 1.f); break;
      case 3: a0 = (float)(unif() * 100.0); break;
      default: a0 = ldexpf(1.0f, (int)(next_u64() % 30) - 15) * (1.0f - ldexpf(1.0f, -24)); break;
    }
    const float want = seq_fold(a0, x);
    expect(same(emulate_terms(a0, x), want), "terms", trial);
    // the same sequence as runs of length one through run_walk
    float r = a0;
    for (float v : x) r = run_walk(r, v, 1u);
    expect(same(r, want), "run_walk m=1", trial);
    // the composition is associative: fold the maps in two halves
    if (n >= 2) {
      const float mid = seq_fold(a0, std::vector<float>(x.begin(), x.begin() + n / 2));
      expect(same(seq_fold(mid, std::vector<float>(x.begin() + n / 2, x.end())), want), "split", trial);
    }
  }
  // 2. runs of equal terms
  for (int trial = 0; trial < 20000; ++trial) {
    const int runs = 1 + (int)(next_u64() % 12);
    float a0 = (trial % 3 == 0) ? -0.0f : (float)(unif() * ldexpf(1.0f, (int)(next_u64() % 16) - 8));
    float seq = a0, emu = a0;
    for (int r = 0; r < runs; ++r) {
      const uint32_t m = 1u + (uint32_t)(next_u64() % (trial % 4 == 0 ? 100000u : 3000u));
      float v = term((int)(next_u64() % 6), ldexpf(1.0f, (int)(next_u64() % 12) - 8));
      if (trial % 5 == 0) {  // exact half ulps of the running sum
        const int e = binade(seq);
        v = ldexpf((float)(2 * (next_u64() % 5) + 1), e - 151);
      }
      for (uint32_t c = 0; c < m; ++c) seq = seq + v;
      emu = run_walk(emu, v, m);
      expect(same(emu, seq), "run_walk", trial);
      emu = seq;  // keep the cases independent
    }
  }
  // 3. run_find against a sequential search
  for (int trial = 0; trial < 20000; ++trial) {
    const float a0 = (trial % 4 == 0) ? 0.f : (float)(unif() * 4.0);
    const float v = term((int)(next_u64() % 6), ldexpf(1.0f, (int)(next_u64() % 10) - 8));
    const uint32_t m = 1u + (uint32_t)(next_u64() % 5000u);
    // a threshold on or near a value the fold takes
    float probe = a0;
    const uint32_t k = (uint32_t)(next_u64() % (m + 1));
    for (uint32_t c = 0; c < k; ++c) probe = probe + v;
    float theta = probe;
    switch (trial % 4) {
      case 1: theta = nextafterf(probe, 0.f); break;
      case 2: theta = nextafterf(probe, INFINITY); break;
      case 3: theta = (float)(unif() * (probe + 1.0f)); break;
    }
    for (int strict = 0; strict < 2; ++strict) {
      uint32_t want = kNone;
      float want_before = 0.f, s = a0;
      for (uint32_t c = 1; c <= m; ++c) {
        const float prev = s;
        s = s + v;
        if (strict ? (s > theta) : (s >= theta)) {
          want = c;
          want_before = prev;
          break;
        }
      }
      float before = -1.f;
      const uint32_t got = strict ? run_find<true>(a0, v, m, theta, &before)
                                  : run_find<false>(a0, v, m, theta, &before);
      expect(got == want, strict ? "run_find >" : "run_find >=", trial);
      if (got == want && want != kNone) expect(same(before, want_before), "run_find before", trial);
    }
  }
  printf("cases %lld mismatches %lld\n", g_cases, g_bad);
  return g_bad != 0;
}
