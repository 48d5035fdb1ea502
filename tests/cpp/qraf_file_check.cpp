// qraf_file_check -- runs the library's .qraf parser (qraf_amd/csrc/qraf_file.cpp,
// the host code behind qraf_file_read_config and qraf_engine_create_from_file)
// over files named on the command line, built with the host sanitizers
// (tests/cpp/Makefile).  Per file one line: the status, the tensor count and
// a checksum over every parsed field and over the first and last byte of each
// tensor's data in the mapping, so every pointer the parser hands out is read.
#include <stdio.h>

#include "../../qraf_amd/csrc/qraf_file.h"

int main(int argc, char** argv) {
    for (int i = 1; i < argc; i++) {
        uint64_t sum = 0;
        size_t nt = 0;
        int rc;
        {
            qraf_hip::Mapping m;
            qraf_hip::Parsed p;
            rc = qraf_hip::map_file(argv[i], m);
            if (rc == QRAF_HIP_OK) rc = qraf_hip::parse(m, p);
            if (rc == QRAF_HIP_OK) {
                const qraf_model_config& c = p.cfg;
                sum = c.vocab_size + 3ull * c.hidden_size + 5ull * c.num_layers + 7ull * c.num_heads +
                      11ull * c.num_kv_heads + 13ull * c.intermediate_size + 17ull * c.max_seq_len +
                      (uint64_t)(c.rope_theta * 1000) + (uint64_t)(c.rms_norm_eps * 1e9) + p.arch.size();
                nt = p.tensors.size();
                for (const qraf_hip::ParsedTensor& t : p.tensors) {
                    sum = sum * 31 + t.name.size() + t.dtype + t.block_size + t.ndim + t.bytes;
                    for (uint32_t d = 0; d < t.ndim; d++) sum = sum * 7 + t.shape[d];
                    if (t.bytes) sum += t.data[0] + 3u * t.data[t.bytes - 1];
                }
                sum += qraf_hip::llama_family(p.arch);
            }
        }
        printf("%d %zu %llu\n", rc, nt, (unsigned long long)sum);
    }
    return 0;
}
