// Host-side model description for the device engine: GGUF metadata, the reference's
// ModelConfig resolution and weight-name resolution, and the HBM-resident weight table.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "iek_internal.h"

namespace iek {

// GGUF metadata value (src/model_loader/gguf_types.rs:4-36).
struct MetaValue {
  uint32_t type = 0;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0;
  float f32 = 0;
  bool b = false;
  std::string s;
  std::vector<MetaValue> arr;
};

struct TensorMeta {
  std::string name;
  std::vector<size_t> dims;
  uint32_t ggml_type = 0;
  uint64_t offset = 0;
};

struct GgufFile {
  uint32_t version = 0;
  std::map<std::string, MetaValue> kv;
  std::vector<TensorMeta> tensors;
  uint64_t data_offset = 0;
  const MetaValue* meta(const std::string& k) const {
    auto it = kv.find(k);
    return it == kv.end() ? nullptr : &it->second;
  }
  const TensorMeta* tensor(const std::string& n) const {
    for (auto& t : tensors)
      if (t.name == n) return &t;
    return nullptr;
  }
};

GgufFile read_gguf(const std::string& path);

enum Family : int { FAM_MISTRAL_LLAMA = 0, FAM_GEMMA4 = 1 };

struct LayerSpec {
  int window = -1;  // -1: full causal
  float rope_theta = 10000.f;
  int rotary_dim = 0;
  int kv_borrow = -1;
  int q_dim = 0, kv_dim = 0, head_dim = 0, ffn_dim = 0;
};

struct Config {
  int family = FAM_MISTRAL_LLAMA;
  int context_length = 0, hidden = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, ffn_dim = 0;
  int vocab = 0;
  float rope_theta = 10000.f, rms_eps = 0.f;
  bool unpack_qk = false;
  std::vector<LayerSpec> layers;
  float embed_scale = 1.f;
  int ple_dim = 0;
  float ple_combine_scale = 0.f, ple_proj_scale = 0.f;
  bool has_softcap = false;
  float softcap = 0.f;
  // TokenizerPromptConfig (src/model_config.rs:8-60)
  bool add_bos = false, add_eos = false;
  uint32_t bos_id = 1, eos_id = 2;
};

Config config_from_gguf(const GgufFile& g);

// A weight resident in HBM in its GGUF byte layout (BF16 is widened to F32 at load like the
// reference's tensor_loader.rs:39-54).
struct DevTensor {
  int dtype = DT_F32;  // iek dtype id (0 F32, 1 Q4K, 2 Q6K, 3 Q8_0)
  std::vector<size_t> dims;
  size_t bytes = 0;
  void* dev = nullptr;
  void* dev_r = nullptr;        // regrouped copy for the decode matvec (Q6_K, Q8_0), or null
  int dtype_r = -1;             // its layout: DT_Q6K_R or DT_Q8_0_R
  std::vector<float> host_f32;  // small F32 tensors also kept on the host (norms, scales)
  bool present() const { return dev != nullptr; }
};

struct LayerTensors {
  DevTensor attn_norm, ffn_norm, attn_post_norm, ffn_post_norm, q_norm, k_norm;
  DevTensor wq, wk, wv, wo, gate, up, down;
  DevTensor ple_gate, ple_proj, ple_post_norm, rope_freqs, out_scale;
  float out_scale_value = 1.f;
  bool has_out_scale = false;
  int rope_table = -1;  // index into Model::rope_tables
};

struct RopeTable {
  float theta;
  int rotary_dim;
  const void* ff_key;
  float* dev;  // [ctx][rotary_dim/2][2] (cos, sin)
};

// Wall times of the load stages, named after the cold-start regions of src/bench_metrics.rs:199-296.
struct LoadTimings {
  double gguf_metadata_ms = 0;        // header, KV table and tensor table
  double config_and_resolve_ms = 0;   // ModelConfig + tensor-name resolution
  double tensor_load_ms = 0;          // tensor bytes from the mapped file into HBM
  double weights_build_ms = 0;        // regrouped matvec copies, shape checks, RoPE tables
};

struct Model {
  int device = 0;
  LoadTimings timings;
  Config cfg;
  std::string path;
  void* blob = nullptr;  // one HBM allocation for every weight
  size_t blob_bytes = 0;
  void* blob_r = nullptr;  // regrouped copies of the matvec weights (Q6_K ffn_down/output, Q8_0 matrices)
  DevTensor token_embd, output_norm, lm_head;
  std::vector<LayerTensors> layers;
  DevTensor ple_token_embd, ple_model_proj, ple_proj_norm;
  std::vector<RopeTable> rope_tables;
  std::map<std::string, const DevTensor*> by_name;  // every loaded tensor (GGUFData::get_tensor)
  ~Model();
};

Model* load_model(const std::string& path, int device);

}  // namespace iek
