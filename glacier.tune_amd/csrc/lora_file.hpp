// lora_file.hpp -- the 'LORA' v1 adapter binary (lora_file.cpp) for
// engine.cpp, which exports it as glacier_lora_* (include/glacier_lora_file.h).
// Each call returns a glacier status code; on failure err holds the message.
#pragma once

#include <string>

#include "../../include/glacier_lora_file.h"

namespace glacier {
namespace lora {

int save(const char* path, int32_t layer_count, int32_t rank, float alpha, int32_t n_tensors,
         const char* const* names, const int32_t* dim0, const int32_t* dim1,
         const float* const* data, std::string& err);
int open(const char* path, glacier_lora_header* header, glacier_lora_reader** reader,
         std::string& err);
int next(glacier_lora_reader* r, char* name, int32_t name_cap, int32_t* dim0, int32_t* dim1,
         std::string& err);
int read(glacier_lora_reader* r, float* dst, int32_t transpose, std::string& err);
void close(glacier_lora_reader* r);

}  // namespace lora
}  // namespace glacier
