// quant.cpp - the group-64 weight packer: fp16 weight rows -> int8 / int4 codes with one fp16 scale per 64 weights
// (the format soc_qmm / soc_dequant read). The rule is the reference's only quantizer, QuantizeMatMulRhs8
// (Mac/cpu/header/matrix_ops.h:42-74: scale = max |w| / 127, zero column -> scale 0, code = clamp(round(w *
// (1 / scale)), -127, 127) with round half away from zero), applied per group of 64 along K instead of per column,
// with 7 for 4-bit codes, and the scale stored in fp16: s = fp16(max |w| / Q), codes computed against that s (a
// scale that rounds to 0 makes a zero group), so that dequantization w = code * s reads exactly the s the codes were
// made for.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "soc_hip.h"
#include "status.h"

namespace {

float half_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, f = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (f == 0) {
      bits = sign;
    } else {  // subnormal: f * 2^-24, exact in fp32
      float v = static_cast<float>(f) * 5.9604644775390625e-8f;
      std::memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (f << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (f << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

void quantize_rows(const uint16_t* w, int64_t r0, int64_t r1, int64_t K, int bits, uint8_t* codes, uint16_t* scales) {
  const int Q = bits == 8 ? 127 : 7;
  const int64_t G = K / 64;
  for (int64_t n = r0; n < r1; ++n) {
    for (int64_t g = 0; g < G; ++g) {
      float v[64], amax = 0.0f;
      for (int i = 0; i < 64; ++i) {
        v[i] = half_to_float(w[n * K + g * 64 + i]);
        amax = std::max(amax, std::fabs(v[i]));
      }
      uint16_t sb = 0;
      float s = 0.0f;
      if (amax != 0.0f) {
        sb = soc_f64_to_f16_rne(static_cast<double>(amax / static_cast<float>(Q)));  // one rounding of the fp32 value
        s = half_to_float(sb);
        if (s == 0.0f) sb = 0;
      }
      scales[n * G + g] = sb;
      const float inv = s != 0.0f ? 1.0f / s : 0.0f;
      for (int i = 0; i < 64; ++i) {
        const int q = s != 0.0f ? std::clamp(static_cast<int>(std::round(v[i] * inv)), -Q, Q) : 0;
        const int64_t k = g * 64 + i;
        if (bits == 8) {
          codes[n * K + k] = static_cast<uint8_t>(static_cast<int8_t>(q));
        } else {
          uint8_t& b = codes[(n * K + k) / 2];
          const uint8_t nib = static_cast<uint8_t>(q) & 0xFu;
          b = (k & 1) ? static_cast<uint8_t>((b & 0x0Fu) | (nib << 4)) : static_cast<uint8_t>((b & 0xF0u) | nib);
        }
      }
    }
  }
}

}  // namespace

extern "C" int soc_quantize_group(const uint16_t* w, int64_t n, int64_t k, int32_t bits, void* codes,
                                  uint16_t* scales) {
  if (w == nullptr || codes == nullptr || scales == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (bits != 8 && bits != 4) return soc::fail(SOC_ERR_INVALID, "soc_quantize_group: bits must be 8 or 4");
  if (n <= 0 || k <= 0 || k % 64 != 0)
    return soc::fail(SOC_ERR_INVALID, "soc_quantize_group: k must be a positive multiple of 64");
  for (int64_t i = 0; i < n * k; ++i)  // inf / NaN have no scale; the reference's rule is undefined for them
    if ((w[i] & 0x7C00u) == 0x7C00u) return soc::fail(SOC_ERR_INVALID, "soc_quantize_group: weights must be finite");
  uint8_t* c = static_cast<uint8_t*>(codes);
  const unsigned hw = std::thread::hardware_concurrency();
  const int64_t nt = std::min<int64_t>(std::max(1u, std::min(hw, 16u)), n);
  std::vector<std::thread> th;
  for (int64_t t = 0; t < nt; ++t)
    th.emplace_back(quantize_rows, w, n * t / nt, n * (t + 1) / nt, k, bits, c, scales);
  for (auto& t : th) t.join();
  return SOC_OK;
}
