// Shared host-side declarations of libczip_hip (not part of the C-ABI).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/czip_hip.h"

namespace czip {

struct HostTensor {
    std::string dtype;
    std::vector<long long> shape;
    const uint8_t* data = nullptr;
    size_t bytes = 0;
    size_t numel = 0;
};

struct HostModel {
    std::vector<uint8_t> blob;
    std::map<std::string, HostTensor> tensors;
    std::map<std::string, std::string> meta;
    std::vector<czip_layer_desc> layers;
    czip_model_desc desc{};
    size_t exp2_numel = 0, rope_numel = 0;
    const uint8_t* tokenizer = nullptr;
    size_t tokenizer_len = 0;
    std::string tokenizer_codec;
};

czip_status load_czm(const char* path, int32_t kv_mode, HostModel& hm, std::string& err);
uint32_t default_cdf_coef_q24();
uint32_t default_target_total(uint32_t vocab);

}  // namespace czip

struct czip_model {
    czip::HostModel hm;
};
