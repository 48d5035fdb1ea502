// qraf_file.h -- the .qraf file parser (host code, no GPU): QrafModel::load's
// header, directory and config parsing (reference src/qraf/loader.cpp:51-117,
// :133-234; src/qraf/header.cpp:8-45), shared by qraf_file_read_config and
// qraf_engine_create_from_file.  Plain C++ so that it builds and runs under
// the host sanitizers.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

#include "status.h"

namespace qraf_hip {

// A read-only mapping of a whole file.
struct Mapping {
    int fd = -1;
    const uint8_t* p = nullptr;
    uint64_t n = 0;
    Mapping() = default;
    Mapping(const Mapping&) = delete;
    Mapping& operator=(const Mapping&) = delete;
    ~Mapping();  // unmaps and closes
};

struct ParsedTensor {
    std::string name;
    uint32_t dtype, block_size, ndim;
    uint32_t shape[8];
    const uint8_t* data;
    uint64_t bytes;
};

struct Parsed {
    qraf_model_config cfg{};
    std::string arch;
    std::vector<ParsedTensor> tensors;
};

// Maps `path` read-only (at least the 128-byte header's size).
int map_file(const char* path, Mapping& m);
// Checks every section and record against the file and reads the config
// block and the tensor directory (tensor data stays in the mapping).
int parse(const Mapping& m, Parsed& out);
// The architectures Transformer::init runs as LLaMA (types.h:126-130); an
// empty name keeps ModelConfig's default arch_type, LLAMA.
bool llama_family(const std::string& a);

}  // namespace qraf_hip
