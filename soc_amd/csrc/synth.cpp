// synth.cpp - the seeded synthetic-data generator used by tests and benchmarks.
//
// The reference ships no generator (its tests use hand-written literals), so this project defines one:
//   key(seed, name)   = mix64(seed ^ mix64(fnv1a64(name)))        (name = the tensor's Hugging Face name)
//   draw(key, i)      = mix64(key + (i + 1) * 0x9e3779b97f4a7c15)  (mix64 = the SplitMix64 finaliser)
//   normal f16        = NORMAL[draw >> 48] where NORMAL[j] = f16_rne(sigma * Phi^-1((j + 0.5) / 65536))
//   uniform f16 [a,b] = f16_rne(a + (b - a) * ((draw >> 11) * 2^-53))
//   token id in [0,V) = ((draw >> 32) * V) >> 32
//   int8 code         = low byte of draw;  int4 code = low nibble of draw (two's complement, [-8, 7])
// Each element depends only on (seed, name, index), so any slice can be produced independently and in parallel.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <thread>
#include <vector>

#include "soc_hip.h"
#include "status.h"

namespace soc {
namespace synth {

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static uint64_t fnv1a64(const char* s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (; *s; ++s) {
    h ^= static_cast<uint8_t>(*s);
    h *= 0x100000001b3ull;
  }
  return h;
}

static inline uint64_t key_of(uint64_t seed, const char* name) { return mix64(seed ^ mix64(fnv1a64(name))); }
static inline uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9e3779b97f4a7c15ull); }

// binary64 -> binary16 with round-to-nearest-even (nearbyint runs in the default FE_TONEAREST mode).
uint16_t f64_to_f16_rne(double x) {
  const uint16_t sign = std::signbit(x) ? 0x8000 : 0;
  const double a = std::fabs(x);
  if (std::isnan(x)) return 0x7e00;
  if (a >= 65520.0) return sign | 0x7c00;
  if (a < 6.103515625e-05) {  // below 2^-14: subnormal grid of 2^-24
    const double m = std::nearbyint(a * 16777216.0);
    return static_cast<uint16_t>(sign | static_cast<uint16_t>(m));
  }
  int e = 0;
  std::frexp(a, &e);
  int E = e - 1;  // a in [2^E, 2^(E+1))
  double m = std::nearbyint(std::ldexp(a, 10 - E));
  if (m >= 2048.0) {
    m = 1024.0;
    ++E;
  }
  if (E > 15) return sign | 0x7c00;
  return static_cast<uint16_t>(sign | ((E + 15) << 10) | (static_cast<int>(m) - 1024));
}

// Phi^-1(p) by bisection on Phi(x) = erfc(-x / sqrt(2)) / 2 to the last bit of binary64.
static double inv_normal_cdf(double p) {
  double lo = -12.0, hi = 12.0;
  for (int it = 0; it < 200; ++it) {
    const double mid = 0.5 * (lo + hi);
    if (mid == lo || mid == hi) break;
    const double c = 0.5 * std::erfc(-mid / std::sqrt(2.0));
    if (c < p) lo = mid;
    else hi = mid;
  }
  return 0.5 * (lo + hi);
}

static const std::vector<double>& unit_quantiles() {
  static std::vector<double> q;
  static std::once_flag once;
  std::call_once(once, [] {
    q.resize(65536);
    for (int j = 0; j < 32768; ++j) {
      const double z = inv_normal_cdf((j + 0.5) / 65536.0);
      q[j] = z;
      q[65535 - j] = -z;
    }
  });
  return q;
}

static const std::vector<uint16_t>& normal_table(float sigma) {
  static std::mutex mu;
  static std::map<uint32_t, std::vector<uint16_t>> tables;
  uint32_t bits;
  std::memcpy(&bits, &sigma, 4);
  std::lock_guard<std::mutex> lock(mu);
  auto it = tables.find(bits);
  if (it != tables.end()) return it->second;
  const std::vector<double>& q = unit_quantiles();
  std::vector<uint16_t> t(65536);
  for (int j = 0; j < 65536; ++j) t[j] = f64_to_f16_rne(static_cast<double>(sigma) * q[j]);
  return tables.emplace(bits, std::move(t)).first->second;
}

template <typename F>
static void parallel_fill(int64_t n, F f) {
  const int64_t grain = 1 << 20;
  unsigned hw = std::thread::hardware_concurrency();
  int nt = static_cast<int>(std::min<int64_t>(hw == 0 ? 1 : hw, (n + grain - 1) / grain));
  if (nt > 16) nt = 16;
  if (nt <= 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  const int64_t chunk = (n + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const int64_t b = t * chunk, e = std::min(n, b + chunk);
    if (b < e) th.emplace_back([=] { f(b, e); });
  }
  for (auto& t : th) t.join();
}

}  // namespace synth
}  // namespace soc

using namespace soc::synth;

extern "C" {

int soc_synth_normal_f16(uint64_t seed, const char* name, float sigma, int64_t offset, int64_t n, uint16_t* out) {
  if (!name || !out || n < 0 || offset < 0 || !(sigma >= 0.0f)) return soc::fail(SOC_ERR_INVALID, "soc_synth_normal_f16: bad argument");
  const uint64_t key = key_of(seed, name);
  const std::vector<uint16_t>& t = normal_table(sigma);
  parallel_fill(n, [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) out[i] = t[draw(key, static_cast<uint64_t>(offset + i)) >> 48];
  });
  return SOC_OK;
}

int soc_synth_uniform_f16(uint64_t seed, const char* name, float lo, float hi, int64_t offset, int64_t n,
                          uint16_t* out) {
  if (!name || !out || n < 0 || offset < 0 || !(hi >= lo)) return soc::fail(SOC_ERR_INVALID, "soc_synth_uniform_f16: bad argument");
  const uint64_t key = key_of(seed, name);
  const double a = lo, w = static_cast<double>(hi) - static_cast<double>(lo);
  parallel_fill(n, [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) {
      const double u = static_cast<double>(draw(key, static_cast<uint64_t>(offset + i)) >> 11) * 0x1.0p-53;
      out[i] = f64_to_f16_rne(a + w * u);
    }
  });
  return SOC_OK;
}

int soc_synth_tokens(uint64_t seed, const char* name, int32_t vocab, int64_t n, int32_t* out) {
  if (!name || !out || n < 0 || vocab <= 0) return soc::fail(SOC_ERR_INVALID, "soc_synth_tokens: bad argument");
  const uint64_t key = key_of(seed, name);
  for (int64_t i = 0; i < n; ++i)
    out[i] = static_cast<int32_t>(((draw(key, static_cast<uint64_t>(i)) >> 32) * static_cast<uint64_t>(vocab)) >> 32);
  return SOC_OK;
}

int soc_synth_int_uniform(uint64_t seed, const char* name, int32_t lo, int32_t hi, int64_t n, int32_t* out) {
  if (!name || !out || n < 0 || hi < lo) return soc::fail(SOC_ERR_INVALID, "soc_synth_int_uniform: bad argument");
  const uint64_t key = key_of(seed, name);
  const uint64_t span = static_cast<uint64_t>(static_cast<int64_t>(hi) - lo + 1);
  for (int64_t i = 0; i < n; ++i)
    out[i] = lo + static_cast<int32_t>(((draw(key, static_cast<uint64_t>(i)) >> 32) * span) >> 32);
  return SOC_OK;
}

int soc_synth_codes(uint64_t seed, const char* name, int32_t bits, int64_t n_codes, uint8_t* out) {
  if (!name || !out || n_codes < 0 || (bits != 8 && bits != 4) || (bits == 4 && n_codes % 2 != 0))
    return soc::fail(SOC_ERR_INVALID, "soc_synth_codes: bad argument");
  const uint64_t key = key_of(seed, name);
  if (bits == 8) {
    parallel_fill(n_codes, [&](int64_t b, int64_t e) {
      for (int64_t i = b; i < e; ++i) out[i] = static_cast<uint8_t>(draw(key, static_cast<uint64_t>(i)) & 0xff);
    });
  } else {
    parallel_fill(n_codes / 2, [&](int64_t b, int64_t e) {
      for (int64_t i = b; i < e; ++i) {
        const uint8_t lo = draw(key, static_cast<uint64_t>(2 * i)) & 0xf;
        const uint8_t hi = draw(key, static_cast<uint64_t>(2 * i + 1)) & 0xf;
        out[i] = static_cast<uint8_t>(lo | (hi << 4));
      }
    });
  }
  return SOC_OK;
}

uint16_t soc_f64_to_f16_rne(double x) { return f64_to_f16_rne(x); }

}  // extern "C"
