/*
 * fence/gguf_parser.hpp -- GGUF v2/v3 reader with the reference's interface
 * (src/gguf/gguf_parser.h:28-217): the same class, enum and member names, so
 * the reference's model code (src/model/qwen3.cu:116-230) compiles against it
 * unchanged.  The file is memory-mapped read-only; tensor data pointers point
 * into the mapping.
 *
 * Behaviour kept from the reference (src/gguf/gguf_parser.cpp):
 *   - versions 2 and 3; magic "GGUF";
 *   - array-valued metadata is skipped and not stored (find_metadata returns
 *     nullptr for it);
 *   - "general.alignment" (u32, non-zero) overrides the default 32;
 *   - at most 4 dims per tensor, unused dims read as 1;
 *   - data_size_bytes = ceil(elements / block_size) * type_size, an unknown
 *     tensor type counting as {1, 4} with a warning;
 *   - get_* throw std::runtime_error when the key is missing or has another
 *     type; find_* return nullptr when absent; open() returns false and
 *     prints the reason on stderr.
 * Checks added (a malformed file is rejected instead of read past its end):
 *   - every length is bounds-checked before use (a string or array longer
 *     than the rest of the file is an error);
 *   - counts larger than the file could hold are rejected before reserving;
 *   - arrays nest at most 16 deep;
 *   - a tensor's data must end inside the file (the reference checks only its
 *     first byte, src/gguf/gguf_parser.cpp:329-335).
 */
#ifndef FENCE_GGUF_PARSER_HPP
#define FENCE_GGUF_PARSER_HPP

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

/* Tensor types; the numbering is the GGUF format's (src/gguf/gguf_parser.h:28-61). */
enum class GGMLType : uint32_t {
    F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q8_1 = 9,
    Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15,
    IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19, IQ4_NL = 20, IQ3_S = 21,
    IQ2_S = 22, IQ4_XS = 23, I8 = 24, I16 = 25, I32 = 26, I64 = 27, F64 = 28,
    IQ1_M = 29, BF16 = 30, TQ1_0 = 34, TQ2_0 = 35, MXFP4 = 39,
};

/* Metadata value types; the numbering is the GGUF format's
 * (src/gguf/gguf_parser.h:64-78). */
enum class GGUFValueType : uint32_t {
    UINT8 = 0, INT8 = 1, UINT16 = 2, INT16 = 3, UINT32 = 4, INT32 = 5, FLOAT32 = 6,
    BOOL = 7, STRING = 8, ARRAY = 9, UINT64 = 10, INT64 = 11, FLOAT64 = 12,
};

struct GGMLTypeInfo {
    uint32_t block_size;  // elements per block
    uint32_t type_size;   // bytes per block
};

/* src/gguf/gguf_parser.h:81-90 */
GGMLTypeInfo ggml_type_info(GGMLType type);
const char* ggml_type_name(GGMLType type);

/* src/gguf/gguf_parser.h:93-108 */
struct GGUFTensorInfo {
    std::string name;
    uint32_t n_dims;
    uint64_t dims[4];  // dims[0] is the contiguous one (a matrix's row length)
    GGMLType type;
    uint64_t offset;   // relative to the start of the tensor data region
    const void* data;  // into the mapping
    size_t data_size_bytes;

    uint64_t n_elements() const {
        uint64_t n = 1;
        for (uint32_t i = 0; i < n_dims; ++i) n *= dims[i];
        return n;
    }
};

/* src/gguf/gguf_parser.h:111-127 (arrays are not stored) */
using GGUFMetadataValue = std::variant<uint8_t, int8_t, uint16_t, int16_t, uint32_t, int32_t, float,
                                       bool, std::string, uint64_t, int64_t, double>;

struct GGUFMetadataKV {
    std::string key;
    GGUFValueType type;
    GGUFMetadataValue value;
};

/* src/gguf/gguf_parser.h:130-217 */
class GGUFFile {
public:
    GGUFFile() = default;
    ~GGUFFile();
    GGUFFile(const GGUFFile&) = delete;
    GGUFFile& operator=(const GGUFFile&) = delete;
    GGUFFile(GGUFFile&& other) noexcept;
    GGUFFile& operator=(GGUFFile&& other) noexcept;

    bool open(const std::string& path);
    void close();
    bool is_open() const { return map_ != nullptr; }

    uint32_t version() const { return version_; }
    uint64_t tensor_count() const { return tensor_count_; }
    uint64_t metadata_count() const { return metadata_count_; }

    const std::vector<GGUFMetadataKV>& metadata() const { return metadata_; }
    const GGUFMetadataKV* find_metadata(const std::string& key) const;
    std::string get_string(const std::string& key) const;
    uint32_t get_u32(const std::string& key) const;
    int32_t get_i32(const std::string& key) const;
    float get_f32(const std::string& key) const;
    bool get_bool(const std::string& key) const;
    uint64_t get_u64(const std::string& key) const;

    const std::vector<GGUFTensorInfo>& tensors() const { return tensors_; }
    const GGUFTensorInfo* find_tensor(const std::string& name) const;

    const std::string& path() const { return path_; }
    size_t file_size() const { return file_size_; }
    size_t data_offset() const { return data_offset_; }
    uint32_t alignment() const { return alignment_; }

    /* Why the last open() failed ("" after a successful one). */
    const std::string& last_error() const { return error_; }

private:
    std::string path_;
    std::string error_;
    void* map_ = nullptr;
    size_t file_size_ = 0;
    int fd_ = -1;
    uint32_t version_ = 0;
    uint64_t tensor_count_ = 0;
    uint64_t metadata_count_ = 0;
    uint32_t alignment_ = 32;
    size_t data_offset_ = 0;
    std::vector<GGUFMetadataKV> metadata_;
    std::vector<GGUFTensorInfo> tensors_;
    std::unordered_map<std::string, size_t> metadata_index_;
    std::unordered_map<std::string, size_t> tensor_index_;

    bool fail(const std::string& why);
    void parse();  // throws on a malformed file
    const GGUFMetadataKV& typed(const std::string& key, GGUFValueType type, const char* what) const;
};

#endif /* FENCE_GGUF_PARSER_HPP */
