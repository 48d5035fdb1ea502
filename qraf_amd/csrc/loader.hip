// loader.hip -- a QRAF file straight into an engine's HBM.
//
// Host code.  Replaces QrafModel::load (reference src/qraf/loader.cpp:51-117)
// followed by Transformer::init's weight binding (src/nn/transformer.cpp:
// 310-439), for the LLaMA-family architectures the engine runs (llama, qwen2,
// mistral).  The file is mapped read-only and parsed by qraf_file.cpp; each
// tensor is copied from the mapping into HBM once by qraf_engine_set_tensor;
// nothing of the file is kept on the host afterwards.  The tied head needs no
// f32 copy of the embedding: the engine's head reads the quantized embedding
// rows (the reference expands them to 1.24 GB of f32 for Qwen2.5-3B,
// transformer.cpp:392-400).
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "qraf_file.h"
#include "qraf_hip.h"

using namespace qraf_hip;

extern "C" {

int qraf_engine_create_from_file(const char* path, const qraf_engine_options* options, qraf_engine** engine) {
    clear_error();
    QH_REQUIRE(engine, QRAF_HIP_ERR_INVALID, "qraf file: null engine pointer");
    *engine = nullptr;
    Mapping m;
    QH_TRY(map_file(path, m));
    Parsed p;
    QH_TRY(parse(m, p));
    QH_REQUIRE(llama_family(p.arch), QRAF_HIP_ERR_INVALID,
               "qraf file: architecture '%s' is not run by this engine (llama, qwen2, mistral)", p.arch.c_str());
    // Each tensor is staged through one pinned host buffer (the largest
    // tensor's size): a copy out of the mapping, then a DMA from pinned memory,
    // instead of the runtime's page-at-a-time pinning of the mapped pages.
    uint64_t big = 0;
    for (const ParsedTensor& t : p.tensors) big = std::max(big, t.bytes);
    void* pin = nullptr;
    if (big) QH_CHECK_HIP(hipHostMalloc(&pin, big, hipHostMallocDefault));
    qraf_engine* e = nullptr;
    int rc = qraf_engine_create(&p.cfg, options, &e);
    for (size_t i = 0; rc == QRAF_HIP_OK && i < p.tensors.size(); i++) {
        const ParsedTensor& t = p.tensors[i];
        memcpy(pin, t.data, t.bytes);
        rc = qraf_engine_set_tensor(e, t.name.c_str(), t.dtype, t.block_size, t.shape, t.ndim, pin, t.bytes);
    }
    if (pin) (void)hipHostFree(pin);
    if (rc != QRAF_HIP_OK) {
        qraf_engine_destroy(e);  // set_tensor's (or create's) message stays the last error
        return rc;
    }
    rc = qraf_engine_finalize(e);
    if (rc != QRAF_HIP_OK) {
        qraf_engine_destroy(e);
        return rc;
    }
    *engine = e;
    return QRAF_HIP_OK;
}

}  // extern "C"
