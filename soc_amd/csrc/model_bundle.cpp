// model_bundle.cpp - soc_model_load_bundle: a bundle on disk into a model on the device (QwenModelLoader::
// LoadModelFromFile, Mac/cpu/src/qwen_model_loader.cpp:35-97): the manifest and its config are validated, then every
// weight the config needs is read (float32 / float16 / bfloat16 files, kept as fp16) and uploaded.
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "soc/assets.h"
#include "soc_hip.h"
#include "status.h"

extern "C" int soc_model_load_bundle(soc_ctx* ctx, const char* manifest_path, soc_model** out) {
  if (ctx == nullptr || manifest_path == nullptr || out == nullptr)
    return soc::fail(SOC_ERR_INVALID, "null argument");
  *out = nullptr;
  soc::ManifestData manifest;
  soc::Qwen3Config config;
  try {
    manifest = soc::ManifestLoader::LoadFromFile(manifest_path);
    config = soc::StartupValidator::ValidateManifest(manifest);
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
  soc_bundle* b = nullptr;  // the C view of the same config (field conversions in one place)
  int rc = soc_bundle_open(manifest_path, &b);
  if (rc != SOC_OK) return rc;
  soc_qwen_config cfg;
  rc = soc_bundle_config(b, &cfg);
  soc_bundle_close(b);
  if (rc != SOC_OK) return rc;
  soc_model* m = nullptr;
  if ((rc = soc_model_create(ctx, &cfg, &m)) != SOC_OK) return rc;
  try {
    for (const auto& [name, shape] : soc::Qwen3TensorShapes(config)) {
      const std::vector<uint16_t> v = soc::WeightLoader::LoadFloat16(manifest, name, shape);
      if ((rc = soc_model_load_tensor(m, name.c_str(), v.data(), static_cast<int64_t>(v.size()))) != SOC_OK) {
        soc_model_destroy(m);
        return rc;
      }
    }
  } catch (const std::exception& e) {
    soc_model_destroy(m);
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
  if ((rc = soc_model_finalize(m)) != SOC_OK) {
    soc_model_destroy(m);
    return rc;
  }
  *out = m;
  return SOC_OK;
}
