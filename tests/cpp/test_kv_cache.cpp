// KVCache through the reference's interface (Mac/gpu/include/runtime/kv_cache.h; kv_cache.mm): creation checks,
// Reserve, AppendPrefill / AppendDecodeToken of fp32 and fp16 rows, per-layer lengths, ViewForLayer contents
// (fp16 planes [kv_head][capacity][head_dim]) and the error messages of kv_cache.mm.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "soc/gpu/runtime.h"

using namespace soc::gpu;

static int fails = 0;
#define EXPECT(cond, msg)                      \
  do {                                         \
    if (!(cond)) {                             \
      std::fprintf(stderr, "FAIL: %s\n", msg); \
      ++fails;                                 \
    }                                          \
  } while (0)

// fp32 -> fp16, round to nearest even (the float is exact in double; the library's converter rounds once)
static uint16_t to_f16_bits(float f) { return soc_f64_to_f16_rne(static_cast<double>(f)); }

int main() {
  std::string err;
  auto ctx = MetalContext::CreateDefault("", "", &err);
  if (!ctx) {
    std::fprintf(stderr, "no HIP context: %s\n", err.c_str());
    return 2;
  }
  EXPECT(KVCache::CreateShared(*ctx, 0, 2, 128, 8, "kv", &err) == nullptr, "zero layers must fail");
  EXPECT(err == "KVCache dimensions must be non-zero", "zero-dimension message");
  const std::size_t L = 2, nkv = 2, hd = 128, cap = 8, W = nkv * hd;
  auto kv = KVCache::CreateShared(*ctx, L, nkv, hd, cap, "kv", &err);
  EXPECT(kv != nullptr, err.c_str());
  if (!kv) return 1;
  EXPECT(kv->GetLayerCount() == L && kv->GetKeyValueHeadCount() == nkv && kv->GetHeadDim() == hd &&
             kv->GetMaxSequenceLength() == cap,
         "dimensions");
  EXPECT(kv->Reserve(cap, &err), "reserve within capacity");
  EXPECT(!kv->Reserve(cap + 1, &err) && err == "KVCache reserve length exceeds max_sequence_length", "reserve beyond");

  // three fp32 rows into layer 0, then one fp16 row (decode) into layer 0 and three fp32 rows into layer 1
  std::vector<float> k3(3 * W), v3(3 * W);
  for (std::size_t i = 0; i < k3.size(); ++i) {
    k3[i] = std::sin(0.37f * i) * 3.0f + 0.001f * i;
    v3[i] = std::cos(0.11f * i) * 2.0f;
  }
  auto kb = MetalBuffer::CreateShared(*ctx, k3.size() * 4, "k", &err);
  auto vb = MetalBuffer::CreateShared(*ctx, v3.size() * 4, "v", &err);
  EXPECT(kb && vb && kb->Write(k3.data(), k3.size() * 4, 0, &err) && vb->Write(v3.data(), v3.size() * 4, 0, &err),
         err.c_str());
  const DeviceTensor kt(kb, 0, TensorDesc::CreateContiguous(DataType::kFloat32, {3, W}));
  const DeviceTensor vt(vb, 0, TensorDesc::CreateContiguous(DataType::kFloat32, {3, W}));
  EXPECT(kv->AppendPrefill(*ctx, 0, kt, vt, &err), err.c_str());
  EXPECT(kv->ViewForLayer(0).sequence_length == 3 && kv->ViewForLayer(1).sequence_length == 0, "per-layer lengths");
  std::vector<uint16_t> k1(W), v1(W);
  for (std::size_t i = 0; i < W; ++i) {
    k1[i] = to_f16_bits(-1.5f + 0.01f * i);
    v1[i] = to_f16_bits(0.25f * (i % 7));
  }
  auto kb1 = MetalBuffer::CreateShared(*ctx, W * 2, "k1", &err);
  auto vb1 = MetalBuffer::CreateShared(*ctx, W * 2, "v1", &err);
  EXPECT(kb1->Write(k1.data(), W * 2, 0, &err) && vb1->Write(v1.data(), W * 2, 0, &err), err.c_str());
  const DeviceTensor kt1(kb1, 0, TensorDesc::CreateContiguous(DataType::kFloat16, {1, W}));
  const DeviceTensor vt1(vb1, 0, TensorDesc::CreateContiguous(DataType::kFloat16, {1, W}));
  EXPECT(kv->AppendDecodeToken(*ctx, 0, kt1, vt1, &err), err.c_str());
  EXPECT(!kv->AppendDecodeToken(*ctx, 1, kt, vt, &err) &&
             err == "KVCache decode append expects single-row key/value tensors",
         "decode append of 3 rows must fail");
  EXPECT(kv->AppendPrefill(*ctx, 1, kt, vt, &err), err.c_str());
  EXPECT(kv->ViewForLayer(0).sequence_length == 4 && kv->ViewForLayer(1).sequence_length == 3, "lengths after");
  EXPECT(!kv->AppendPrefill(*ctx, 2, kt, vt, &err) && err == "KVCache layer index is out of range", "layer range");
  const DeviceTensor narrow(kb, 0, TensorDesc::CreateContiguous(DataType::kFloat32, {3, W / 2}));
  EXPECT(!kv->AppendPrefill(*ctx, 1, narrow, narrow, &err) &&
             err == "KVCache append tensor hidden size does not match cache configuration",
         "width check");
  EXPECT(kv->AppendPrefill(*ctx, 0, kt, vt, &err), "4 + 3 rows fit in 8");
  EXPECT(!kv->AppendPrefill(*ctx, 0, kt, vt, &err) && err == "KVCache append would exceed max_sequence_length",
         "capacity");
  EXPECT(kv->ViewForLayer(0).sequence_length == 7, "a failed append leaves the length");
  err.clear();

  // contents of layer 0: rows 0..2 from k3 (rounded to fp16), row 3 = k1
  const KVCacheLayerView view = kv->ViewForLayer(0);
  const auto& st = view.keys.GetDesc().GetStrides();
  EXPECT(view.keys.GetDesc().GetDataType() == DataType::kFloat16 && st.size() == 3 && st[0] == cap * hd &&
             st[1] == hd && st[2] == 1,
         "view layout");
  std::vector<uint16_t> plane(nkv * cap * hd);
  EXPECT(view.keys.GetBuffer()->Read(plane.data(), plane.size() * 2, view.keys.GetByteOffset(), &err), err.c_str());
  int bad = 0;
  for (std::size_t h = 0; h < nkv; ++h)
    for (std::size_t p = 0; p < 4; ++p)
      for (std::size_t d = 0; d < hd; ++d) {
        const uint16_t want = p < 3 ? to_f16_bits(k3[p * W + h * hd + d]) : k1[h * hd + d];
        bad += plane[(h * cap + p) * hd + d] != want;
      }
  EXPECT(bad == 0, "layer 0 key plane contents");
  if (fails == 0) std::printf("test_kv_cache passed\n");
  return fails == 0 ? 0 : 1;
}
