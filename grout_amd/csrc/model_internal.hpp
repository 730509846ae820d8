// The loaded-model object behind grout_model (include/grout_engine.h), shared
// by the safetensors loader (loader.cpp) and the GGUF loader (gguf.cpp).
#pragma once

#include <string>
#include <vector>

#include "../../include/grout_engine.h"

struct grout_model {
  grout_model_info info{};
  int device = 0;
  void* arena = nullptr;  // every weight, one device allocation
  // fp16 checkpoints (safetensors): fused fp16 layouts
  std::vector<grout_qwen3_layer> layers;
  const void* embed = nullptr;
  const void* norm = nullptr;
  const void* lm_head = nullptr;
  // GGUF checkpoints: per-part formats (low-bit parts in the GEMV layout)
  bool low_bit = false;
  std::vector<grout_qwen3_qlayer> qlayers;
  grout_wpart qembed{};
  grout_wpart qlm_head{};
};

namespace grout_gguf {
// A path naming a .gguf file (the reference's is_gguf_path, src/loader.rs).
bool is_gguf_path(const char* path);
// grout_model_inspect / grout_model_load for a GGUF file.
int inspect(const char* path, grout_model_info* info);
int load(const char* path, int device, grout_model** out);
}  // namespace grout_gguf
