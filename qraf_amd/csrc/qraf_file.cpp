// qraf_file.cpp -- the .qraf file parser (host code, no GPU).
//
// Replaces QrafModel::load's parsing (reference src/qraf/loader.cpp:51-117:
// open, mmap, header check, quant / tensor directories, config block).
// File layout (include/qraf/format.h:26-132, little-endian, packed): a
// 128-byte header of section offsets and counts; the config block (u32 count,
// then 12-byte {key string offset, type, value} entries); the tensor directory
// (80-byte entries: name hash, name string offset, ndim, shape[8], dtype,
// quant scheme id, data offset and size, layout); the quant directory (32-byte
// entries: id, type, block size, ...); a string table of NUL-terminated names.
// Every offset is checked against the file before it is read, as
// validate_header (src/qraf/header.cpp:8-45) and get_string (loader.cpp:273-277)
// do, and more strictly: a string must end inside the string table.
#include "qraf_file.h"

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace qraf_hip {
namespace {

constexpr uint32_t FILE_MAGIC = 0x46415251u;  // "QRAF", types.h:24
constexpr uint32_t FILE_VERSION = 1;          // types.h:25

#pragma pack(push, 1)
struct FileHeader {
    uint32_t magic, version;
    uint64_t file_size, config_offset, config_size, tokenizer_offset, tokenizer_size, tensor_dir_offset,
        tensor_dir_size, quant_dir_offset, quant_dir_size, string_table_offset, string_table_size, data_offset;
    uint32_t num_tensors, num_quant_schemes, flags, padding;
    uint8_t reserved[8];
};
struct ConfigRecord {
    uint32_t key_offset, value_type, value;
};
struct TensorRecord {
    uint64_t name_hash;
    uint32_t name_offset, ndim, shape[8], dtype, quant_scheme_id;
    uint64_t data_offset, data_size;
    uint32_t layout_id, padding;
};
struct SchemeRecord {
    uint32_t id, type, block_size, group_size;
    float scale, zero_point;
    uint32_t flags, padding;
};
#pragma pack(pop)
static_assert(sizeof(FileHeader) == 128, "QRAF header is 128 bytes");
static_assert(sizeof(ConfigRecord) == 12, "config entry is 12 bytes");
static_assert(sizeof(TensorRecord) == 80, "tensor entry is 80 bytes");
static_assert(sizeof(SchemeRecord) == 32, "quant scheme entry is 32 bytes");

// [off, off + len) inside a file of n bytes, without overflow
bool within(uint64_t off, uint64_t len, uint64_t n) { return off <= n && len <= n - off; }

// NUL-terminated string at `off` of the string table
int table_string(const Mapping& m, const FileHeader& h, uint32_t off, std::string& out) {
    QH_REQUIRE(off < h.string_table_size, QRAF_HIP_ERR_FORMAT, "qraf file: string offset %u out of bounds", off);
    const char* s = (const char*)m.p + h.string_table_offset + off;
    const size_t room = (size_t)(h.string_table_size - off);
    const size_t len = strnlen(s, room);
    QH_REQUIRE(len < room, QRAF_HIP_ERR_FORMAT, "qraf file: string at %u not terminated in the table", off);
    out.assign(s, len);
    return QRAF_HIP_OK;
}

}  // namespace

Mapping::~Mapping() {
    if (p) munmap(const_cast<uint8_t*>(p), n);
    if (fd >= 0) close(fd);
}

int map_file(const char* path, Mapping& m) {
    QH_REQUIRE(path, QRAF_HIP_ERR_INVALID, "qraf file: null path");
    m.fd = open(path, O_RDONLY);
    QH_REQUIRE(m.fd >= 0, QRAF_HIP_ERR_INVALID, "qraf file: cannot open %s", path);
    struct stat st;
    QH_REQUIRE(fstat(m.fd, &st) == 0, QRAF_HIP_ERR_INVALID, "qraf file: cannot stat %s", path);
    m.n = (uint64_t)st.st_size;
    QH_REQUIRE(m.n >= sizeof(FileHeader), QRAF_HIP_ERR_FORMAT, "qraf file: %llu bytes, too small for the header",
               (unsigned long long)m.n);
    void* p = mmap(nullptr, m.n, PROT_READ, MAP_PRIVATE | MAP_POPULATE, m.fd, 0);
    QH_REQUIRE(p != MAP_FAILED, QRAF_HIP_ERR_INVALID, "qraf file: mmap of %s failed", path);
    m.p = (const uint8_t*)p;
    madvise(p, m.n, MADV_SEQUENTIAL);  // as loader.cpp:90
    return QRAF_HIP_OK;
}

int parse(const Mapping& m, Parsed& out) {
    FileHeader h;
    memcpy(&h, m.p, sizeof h);
    // header.cpp:8-45
    QH_REQUIRE(h.magic == FILE_MAGIC, QRAF_HIP_ERR_FORMAT, "qraf file: magic 0x%08X (expected 0x%08X)", h.magic,
               FILE_MAGIC);
    QH_REQUIRE(h.version == FILE_VERSION, QRAF_HIP_ERR_FORMAT, "qraf file: version %u (expected %u)", h.version,
               FILE_VERSION);
    QH_REQUIRE(h.file_size == m.n, QRAF_HIP_ERR_FORMAT, "qraf file: header says %llu bytes, file has %llu",
               (unsigned long long)h.file_size, (unsigned long long)m.n);
    QH_REQUIRE(within(h.config_offset, h.config_size, m.n), QRAF_HIP_ERR_FORMAT,
               "qraf file: config block extends past the file");
    QH_REQUIRE(within(h.tensor_dir_offset, h.tensor_dir_size, m.n), QRAF_HIP_ERR_FORMAT,
               "qraf file: tensor directory extends past the file");
    QH_REQUIRE(within(h.quant_dir_offset, h.quant_dir_size, m.n), QRAF_HIP_ERR_FORMAT,
               "qraf file: quant directory extends past the file");
    QH_REQUIRE(within(h.string_table_offset, h.string_table_size, m.n), QRAF_HIP_ERR_FORMAT,
               "qraf file: string table extends past the file");
    QH_REQUIRE(h.data_offset <= m.n, QRAF_HIP_ERR_FORMAT, "qraf file: data offset past the file");
    QH_REQUIRE((uint64_t)h.num_tensors * sizeof(TensorRecord) <= h.tensor_dir_size, QRAF_HIP_ERR_FORMAT,
               "qraf file: %u tensors do not fit the tensor directory", h.num_tensors);
    QH_REQUIRE((uint64_t)h.num_quant_schemes * sizeof(SchemeRecord) <= h.quant_dir_size, QRAF_HIP_ERR_FORMAT,
               "qraf file: %u quant schemes do not fit the quant directory", h.num_quant_schemes);

    // quant directory (loader.cpp:222-234)
    std::vector<SchemeRecord> schemes(h.num_quant_schemes);
    if (h.num_quant_schemes)
        memcpy(schemes.data(), m.p + h.quant_dir_offset, (size_t)h.num_quant_schemes * sizeof(SchemeRecord));

    // config block (loader.cpp:133-177), with ModelConfig's defaults (types.h:97-110)
    qraf_model_config& c = out.cfg;
    c = qraf_model_config{0, 0, 0, 0, 0, 0, 2048, 10000.0f, 1e-5f};
    if (h.config_size) {
        QH_REQUIRE(h.config_size >= 4, QRAF_HIP_ERR_FORMAT, "qraf file: config block too small");
        uint32_t ne;
        memcpy(&ne, m.p + h.config_offset, 4);
        QH_REQUIRE((uint64_t)ne * sizeof(ConfigRecord) <= h.config_size - 4, QRAF_HIP_ERR_FORMAT,
                   "qraf file: %u config entries do not fit the config block", ne);
        for (uint32_t i = 0; i < ne; i++) {
            ConfigRecord r;
            memcpy(&r, m.p + h.config_offset + 4 + (uint64_t)i * sizeof r, sizeof r);
            std::string key;
            QH_TRY(table_string(m, h, r.key_offset, key));
            float f;
            memcpy(&f, &r.value, 4);
            if (key == "architecture") QH_TRY(table_string(m, h, r.value, out.arch));
            else if (key == "vocab_size") c.vocab_size = r.value;
            else if (key == "hidden_size") c.hidden_size = r.value;
            else if (key == "num_layers") c.num_layers = r.value;
            else if (key == "num_heads") c.num_heads = r.value;
            else if (key == "num_kv_heads") c.num_kv_heads = r.value;
            else if (key == "intermediate_size") c.intermediate_size = r.value;
            else if (key == "max_seq_len") c.max_seq_len = r.value;
            else if (key == "rope_theta") c.rope_theta = f;
            else if (key == "rms_norm_eps") c.rms_norm_eps = f;
            // other keys are ignored, as by the reference
        }
    }
    if (c.num_kv_heads == 0) c.num_kv_heads = c.num_heads;  // ModelConfig::compute_derived, types.h:121-124

    // tensor directory (loader.cpp:180-220)
    out.tensors.clear();
    out.tensors.reserve(h.num_tensors);
    for (uint32_t i = 0; i < h.num_tensors; i++) {
        TensorRecord r;
        memcpy(&r, m.p + h.tensor_dir_offset + (uint64_t)i * sizeof r, sizeof r);
        ParsedTensor t;
        QH_TRY(table_string(m, h, r.name_offset, t.name));
        QH_REQUIRE(within(r.data_offset, r.data_size, m.n), QRAF_HIP_ERR_FORMAT,
                   "qraf file: tensor '%s' data extends past the file", t.name.c_str());
        QH_REQUIRE(r.ndim >= 1 && r.ndim <= 8, QRAF_HIP_ERR_FORMAT, "qraf file: tensor '%s' has %u dimensions",
                   t.name.c_str(), r.ndim);
        t.dtype = r.dtype;
        t.block_size = 0;
        if (r.quant_scheme_id != 0xFFFFFFFFu && r.quant_scheme_id < schemes.size())
            t.block_size = schemes[r.quant_scheme_id].block_size;
        t.ndim = r.ndim;
        memcpy(t.shape, r.shape, sizeof t.shape);
        t.data = m.p + r.data_offset;
        t.bytes = r.data_size;
        out.tensors.push_back(std::move(t));
    }
    return QRAF_HIP_OK;
}

bool llama_family(const std::string& a) { return a.empty() || a == "llama" || a == "qwen2" || a == "mistral"; }

}  // namespace qraf_hip

extern "C" int qraf_file_read_config(const char* path, qraf_model_config* config, uint32_t* num_tensors) {
    using namespace qraf_hip;
    clear_error();
    QH_REQUIRE(config, QRAF_HIP_ERR_INVALID, "qraf file: null config");
    Mapping m;
    QH_TRY(map_file(path, m));
    Parsed p;
    QH_TRY(parse(m, p));
    *config = p.cfg;
    if (num_tensors) *num_tensors = (uint32_t)p.tensors.size();
    return QRAF_HIP_OK;
}
