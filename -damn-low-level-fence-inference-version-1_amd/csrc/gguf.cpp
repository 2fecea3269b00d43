// gguf.cpp -- GGUF v2/v3 reader (host only), the interface of
// src/gguf/gguf_parser.h with bounds-checked parsing; plus its C ABI
// (include/fence/gguf.h).
//
// Layout of a GGUF file (the format, as src/gguf/gguf_parser.cpp:144-345
// reads it): magic u32 "GGUF", version u32, tensor_count u64, kv_count u64;
// kv_count entries {string key, u32 type, value}; tensor_count entries
// {string name, u32 n_dims, u64 dims[n_dims], u32 type, u64 offset}; then,
// at the next multiple of the alignment, the tensor data region.  Strings are
// u64 length + bytes; arrays are u32 element type + u64 count + elements.
#include "fence/gguf.h"
#include "fence/gguf_parser.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <utility>

GGMLTypeInfo ggml_type_info(GGMLType type) {
    switch (type) {  // {elements per block, bytes per block} of each format
        case GGMLType::F32: return {1, 4};
        case GGMLType::F16: return {1, 2};
        case GGMLType::BF16: return {1, 2};
        case GGMLType::F64: return {1, 8};
        case GGMLType::I8: return {1, 1};
        case GGMLType::I16: return {1, 2};
        case GGMLType::I32: return {1, 4};
        case GGMLType::I64: return {1, 8};
        case GGMLType::Q4_0: return {32, 2 + 16};
        case GGMLType::Q4_1: return {32, 4 + 16};
        case GGMLType::Q5_0: return {32, 2 + 4 + 16};
        case GGMLType::Q5_1: return {32, 4 + 4 + 16};
        case GGMLType::Q8_0: return {32, 2 + 32};
        case GGMLType::Q8_1: return {32, 8 + 32};
        case GGMLType::Q2_K: return {256, 16 + 64 + 4};
        case GGMLType::Q3_K: return {256, 32 + 64 + 12 + 2};
        case GGMLType::Q4_K: return {256, 4 + 12 + 128};
        case GGMLType::Q5_K: return {256, 4 + 12 + 32 + 128};
        case GGMLType::Q6_K: return {256, 128 + 64 + 16 + 2};
        case GGMLType::Q8_K: return {256, 4 + 256 + 32};
        default:
            // src/gguf/gguf_parser.cpp:45-48: unknown types are sized as F32
            std::fprintf(stderr, "WARNING: unknown GGMLType %u, assuming F32\n",
                         static_cast<uint32_t>(type));
            return {1, 4};
    }
}

const char* ggml_type_name(GGMLType type) {
    switch (type) {
        case GGMLType::F32: return "F32";
        case GGMLType::F16: return "F16";
        case GGMLType::Q4_0: return "Q4_0";
        case GGMLType::Q4_1: return "Q4_1";
        case GGMLType::Q5_0: return "Q5_0";
        case GGMLType::Q5_1: return "Q5_1";
        case GGMLType::Q8_0: return "Q8_0";
        case GGMLType::Q8_1: return "Q8_1";
        case GGMLType::Q2_K: return "Q2_K";
        case GGMLType::Q3_K: return "Q3_K";
        case GGMLType::Q4_K: return "Q4_K";
        case GGMLType::Q5_K: return "Q5_K";
        case GGMLType::Q6_K: return "Q6_K";
        case GGMLType::Q8_K: return "Q8_K";
        case GGMLType::BF16: return "BF16";
        case GGMLType::I8: return "I8";
        case GGMLType::I16: return "I16";
        case GGMLType::I32: return "I32";
        case GGMLType::I64: return "I64";
        case GGMLType::F64: return "F64";
        default: return "UNKNOWN";
    }
}

namespace {

struct ParseError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// A cursor that never moves past `end`.
struct Reader {
    const uint8_t* p;
    const uint8_t* end;

    uint64_t left() const { return static_cast<uint64_t>(end - p); }

    void need(uint64_t n, const char* what) const {
        if (n > left()) throw ParseError(std::string("unexpected end of file in ") + what);
    }
    template <class T>
    T get(const char* what) {
        need(sizeof(T), what);
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str(const char* what) {
        const uint64_t n = get<uint64_t>(what);
        need(n, what);
        std::string s(reinterpret_cast<const char*>(p), static_cast<size_t>(n));
        p += n;
        return s;
    }
    void skip(uint64_t n, const char* what) {
        need(n, what);
        p += n;
    }
};

// Bytes of one scalar value of type t, 0 for STRING / ARRAY, -1 if unknown.
int scalar_bytes(GGUFValueType t) {
    switch (t) {
        case GGUFValueType::UINT8:
        case GGUFValueType::INT8:
        case GGUFValueType::BOOL: return 1;
        case GGUFValueType::UINT16:
        case GGUFValueType::INT16: return 2;
        case GGUFValueType::UINT32:
        case GGUFValueType::INT32:
        case GGUFValueType::FLOAT32: return 4;
        case GGUFValueType::UINT64:
        case GGUFValueType::INT64:
        case GGUFValueType::FLOAT64: return 8;
        case GGUFValueType::STRING:
        case GGUFValueType::ARRAY: return 0;
    }
    return -1;
}

constexpr int kMaxArrayDepth = 16;

void skip_array(Reader& r, int depth) {
    if (depth > kMaxArrayDepth) throw ParseError("arrays nested too deep");
    const auto t = r.get<GGUFValueType>("array type");
    const uint64_t n = r.get<uint64_t>("array length");
    const int sb = scalar_bytes(t);
    if (sb < 0) throw ParseError("unknown array element type " + std::to_string(static_cast<uint32_t>(t)));
    if (sb > 0) {  // fixed-size elements: one bounds check
        if (n > r.left() / static_cast<uint64_t>(sb)) throw ParseError("unexpected end of file in array");
        r.skip(n * static_cast<uint64_t>(sb), "array");
        return;
    }
    // strings need at least 8 bytes and arrays 12 each: cap the count first
    if (n > r.left() / 8) throw ParseError("unexpected end of file in array");
    for (uint64_t i = 0; i < n; ++i) {
        if (t == GGUFValueType::STRING) r.skip(r.get<uint64_t>("string length"), "string");
        else skip_array(r, depth + 1);
    }
}

GGUFMetadataValue read_scalar_value(Reader& r, GGUFValueType t) {
    switch (t) {
        case GGUFValueType::UINT8: return r.get<uint8_t>("value");
        case GGUFValueType::INT8: return r.get<int8_t>("value");
        case GGUFValueType::UINT16: return r.get<uint16_t>("value");
        case GGUFValueType::INT16: return r.get<int16_t>("value");
        case GGUFValueType::UINT32: return r.get<uint32_t>("value");
        case GGUFValueType::INT32: return r.get<int32_t>("value");
        case GGUFValueType::FLOAT32: return r.get<float>("value");
        case GGUFValueType::BOOL: return r.get<uint8_t>("value") != 0;
        case GGUFValueType::STRING: return r.str("string value");
        case GGUFValueType::UINT64: return r.get<uint64_t>("value");
        case GGUFValueType::INT64: return r.get<int64_t>("value");
        case GGUFValueType::FLOAT64: return r.get<double>("value");
        case GGUFValueType::ARRAY: break;
    }
    throw ParseError("unknown metadata value type " + std::to_string(static_cast<uint32_t>(t)));
}

}  // namespace

bool GGUFFile::fail(const std::string& why) {
    std::fprintf(stderr, "GGUF: %s\n", why.c_str());
    const std::string keep = why;
    close();
    error_ = keep;
    return false;
}

void GGUFFile::parse() {
    const auto* base = static_cast<const uint8_t*>(map_);
    Reader r{base, base + file_size_};

    const uint32_t magic = r.get<uint32_t>("header");
    if (magic != 0x46554747u) {  // "GGUF" little-endian
        char buf[64];
        std::snprintf(buf, sizeof buf, "invalid magic 0x%08X (expected 0x46554747 'GGUF')", magic);
        throw ParseError(buf);
    }
    version_ = r.get<uint32_t>("header");
    if (version_ < 2 || version_ > 3)
        throw ParseError("unsupported version " + std::to_string(version_) + " (expected 2 or 3)");
    tensor_count_ = r.get<uint64_t>("header");
    metadata_count_ = r.get<uint64_t>("header");
    // an entry takes at least 12 (kv) / 24 (tensor info) bytes
    if (metadata_count_ > r.left() / 12) throw ParseError("metadata count exceeds the file");
    if (tensor_count_ > r.left() / 24) throw ParseError("tensor count exceeds the file");

    metadata_.reserve(static_cast<size_t>(metadata_count_));
    for (uint64_t i = 0; i < metadata_count_; ++i) {
        GGUFMetadataKV kv;
        kv.key = r.str("metadata key");
        kv.type = r.get<GGUFValueType>("metadata type");
        if (kv.type == GGUFValueType::ARRAY) {  // skipped, not stored
            skip_array(r, 1);
            continue;
        }
        kv.value = read_scalar_value(r, kv.type);
        if (kv.key == "general.alignment" && kv.type == GGUFValueType::UINT32) {
            const uint32_t a = std::get<uint32_t>(kv.value);
            if (a == 0)
                std::fprintf(stderr, "GGUF: general.alignment is 0, ignoring (keeping default %u)\n", alignment_);
            else
                alignment_ = a;
        }
        metadata_index_[kv.key] = metadata_.size();
        metadata_.push_back(std::move(kv));
    }

    tensors_.reserve(static_cast<size_t>(tensor_count_));
    for (uint64_t i = 0; i < tensor_count_; ++i) {
        GGUFTensorInfo ti{};
        ti.name = r.str("tensor name");
        ti.n_dims = r.get<uint32_t>("tensor dims");
        if (ti.n_dims > 4)
            throw ParseError("tensor '" + ti.name + "' has " + std::to_string(ti.n_dims) + " dims (max 4)");
        for (uint32_t d = 0; d < 4; ++d) ti.dims[d] = d < ti.n_dims ? r.get<uint64_t>("tensor dims") : 1;
        ti.type = r.get<GGMLType>("tensor type");
        ti.offset = r.get<uint64_t>("tensor offset");
        tensor_index_[ti.name] = tensors_.size();
        tensors_.push_back(std::move(ti));
    }

    const size_t header_end = static_cast<size_t>(r.p - base);
    data_offset_ = header_end + (alignment_ - header_end % alignment_) % alignment_;

    for (auto& ti : tensors_) {
        const GGMLTypeInfo info = ggml_type_info(ti.type);
        // Element count, each multiply checked before it is made (the dims
        // come from the file).  2^72 elements need more than 2^64 bytes in
        // every type (a block of at most 256 elements takes at least one
        // byte), so no file holds them; capping n there keeps it and the byte
        // count below far from wrapping, and the end-of-file check rejects
        // the rest.
        const unsigned __int128 max_n = static_cast<unsigned __int128>(1) << 72;
        unsigned __int128 n = 1;
        for (uint32_t d = 0; d < ti.n_dims; ++d) {
            const uint64_t dim = ti.dims[d];
            if (dim != 0 && n > max_n / dim)
                throw ParseError("tensor '" + ti.name + "' has more elements than the file could hold");
            n *= dim;
        }
        const unsigned __int128 bytes = (n + info.block_size - 1) / info.block_size * info.type_size;
        const unsigned __int128 start = static_cast<unsigned __int128>(data_offset_) + ti.offset;
        if (start >= file_size_)
            throw ParseError("tensor '" + ti.name + "' offset " + std::to_string(static_cast<uint64_t>(start)) +
                             " exceeds file size " + std::to_string(file_size_));
        if (start + bytes > file_size_)
            throw ParseError("tensor '" + ti.name + "' data runs past the end of the file");
        ti.data = base + static_cast<size_t>(start);
        ti.data_size_bytes = static_cast<size_t>(bytes);
    }
}

bool GGUFFile::open(const std::string& path) {
    if (map_ || fd_ >= 0) close();
    error_.clear();
    path_ = path;
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) return fail("cannot open '" + path + "': " + std::strerror(errno));
    struct stat st;
    if (fstat(fd_, &st) != 0) return fail(std::string("fstat failed: ") + std::strerror(errno));
    file_size_ = static_cast<size_t>(st.st_size);
    if (file_size_ == 0) return fail("'" + path + "' is empty");
    void* m = mmap(nullptr, file_size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) return fail(std::string("mmap failed: ") + std::strerror(errno));
    map_ = m;
    madvise(map_, file_size_, MADV_SEQUENTIAL);
    try {
        parse();
    } catch (const std::exception& e) {
        return fail(e.what());
    }
    madvise(map_, file_size_, MADV_RANDOM);
    return true;
}

void GGUFFile::close() {
    if (map_) munmap(map_, file_size_);
    if (fd_ >= 0) ::close(fd_);
    map_ = nullptr;
    fd_ = -1;
    file_size_ = 0;
    version_ = 0;
    tensor_count_ = 0;
    metadata_count_ = 0;
    alignment_ = 32;
    data_offset_ = 0;
    metadata_.clear();
    tensors_.clear();
    metadata_index_.clear();
    tensor_index_.clear();
}

GGUFFile::~GGUFFile() { close(); }

GGUFFile::GGUFFile(GGUFFile&& o) noexcept { *this = std::move(o); }

GGUFFile& GGUFFile::operator=(GGUFFile&& o) noexcept {
    if (this == &o) return *this;
    close();
    path_ = std::move(o.path_);
    error_ = std::move(o.error_);
    map_ = std::exchange(o.map_, nullptr);
    file_size_ = std::exchange(o.file_size_, 0);
    fd_ = std::exchange(o.fd_, -1);
    version_ = o.version_;
    tensor_count_ = o.tensor_count_;
    metadata_count_ = o.metadata_count_;
    alignment_ = o.alignment_;
    data_offset_ = o.data_offset_;
    metadata_ = std::move(o.metadata_);
    tensors_ = std::move(o.tensors_);
    metadata_index_ = std::move(o.metadata_index_);
    tensor_index_ = std::move(o.tensor_index_);
    o.close();
    return *this;
}

const GGUFTensorInfo* GGUFFile::find_tensor(const std::string& name) const {
    const auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

const GGUFMetadataKV* GGUFFile::find_metadata(const std::string& key) const {
    const auto it = metadata_index_.find(key);
    return it == metadata_index_.end() ? nullptr : &metadata_[it->second];
}

const GGUFMetadataKV& GGUFFile::typed(const std::string& key, GGUFValueType type, const char* what) const {
    const GGUFMetadataKV* kv = find_metadata(key);
    if (!kv) throw std::runtime_error("GGUF: metadata key not found: " + key);
    if (kv->type != type) throw std::runtime_error("GGUF: key '" + key + "' is not " + what);
    return *kv;
}

std::string GGUFFile::get_string(const std::string& key) const {
    return std::get<std::string>(typed(key, GGUFValueType::STRING, "a string").value);
}
uint32_t GGUFFile::get_u32(const std::string& key) const {
    return std::get<uint32_t>(typed(key, GGUFValueType::UINT32, "u32").value);
}
int32_t GGUFFile::get_i32(const std::string& key) const {
    return std::get<int32_t>(typed(key, GGUFValueType::INT32, "i32").value);
}
float GGUFFile::get_f32(const std::string& key) const {
    return std::get<float>(typed(key, GGUFValueType::FLOAT32, "f32").value);
}
bool GGUFFile::get_bool(const std::string& key) const {
    return std::get<bool>(typed(key, GGUFValueType::BOOL, "bool").value);
}
uint64_t GGUFFile::get_u64(const std::string& key) const {
    return std::get<uint64_t>(typed(key, GGUFValueType::UINT64, "u64").value);
}

// ------------------------------------------------------------------ C ABI

struct fence_gguf {
    GGUFFile file;
};

namespace {

void fill_info(const GGUFTensorInfo& t, fence_gguf_tensor_info* out) {
    out->name = t.name.c_str();
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->dims[d] = t.dims[d];
    out->type = static_cast<uint32_t>(t.type);
    out->offset = t.offset;
    out->data = t.data;
    out->data_size_bytes = t.data_size_bytes;
}

template <class T, class F>
int get_typed(const fence_gguf* g, const char* key, T* out, GGUFValueType type, F&& conv) {
    if (!g || !key || !out) return FENCE_ERROR_INVALID_VALUE;
    const GGUFMetadataKV* kv = g->file.find_metadata(key);
    if (!kv) return FENCE_ERROR_NOT_FOUND;
    if (kv->type != type) return FENCE_ERROR_TYPE_MISMATCH;
    *out = conv(kv->value);
    return FENCE_SUCCESS;
}

}  // namespace

extern "C" int fence_gguf_open(const char* path, fence_gguf** out, char* err, size_t err_len) {
    if (!path || !out) return FENCE_ERROR_INVALID_VALUE;
    *out = nullptr;
    auto* g = new (std::nothrow) fence_gguf;
    if (!g) return FENCE_ERROR_OUT_OF_MEMORY;
    if (!g->file.open(path)) {
        if (err && err_len) std::snprintf(err, err_len, "%s", g->file.last_error().c_str());
        delete g;
        return FENCE_ERROR_BAD_FILE;
    }
    *out = g;
    return FENCE_SUCCESS;
}

extern "C" void fence_gguf_close(fence_gguf* g) { delete g; }

extern "C" uint32_t fence_gguf_version(const fence_gguf* g) { return g ? g->file.version() : 0; }
extern "C" uint64_t fence_gguf_tensor_count(const fence_gguf* g) { return g ? g->file.tensor_count() : 0; }
extern "C" uint64_t fence_gguf_metadata_count(const fence_gguf* g) { return g ? g->file.metadata_count() : 0; }
extern "C" uint64_t fence_gguf_file_size(const fence_gguf* g) { return g ? g->file.file_size() : 0; }
extern "C" uint64_t fence_gguf_data_offset(const fence_gguf* g) { return g ? g->file.data_offset() : 0; }
extern "C" uint32_t fence_gguf_alignment(const fence_gguf* g) { return g ? g->file.alignment() : 0; }

extern "C" int fence_gguf_find_tensor(const fence_gguf* g, const char* name, fence_gguf_tensor_info* out) {
    if (!g || !name || !out) return FENCE_ERROR_INVALID_VALUE;
    const GGUFTensorInfo* t = g->file.find_tensor(name);
    if (!t) return FENCE_ERROR_NOT_FOUND;
    fill_info(*t, out);
    return FENCE_SUCCESS;
}

extern "C" int fence_gguf_tensor_at(const fence_gguf* g, uint64_t index, fence_gguf_tensor_info* out) {
    if (!g || !out) return FENCE_ERROR_INVALID_VALUE;
    if (index >= g->file.tensors().size()) return FENCE_ERROR_NOT_FOUND;
    fill_info(g->file.tensors()[static_cast<size_t>(index)], out);
    return FENCE_SUCCESS;
}

extern "C" int fence_gguf_metadata_type(const fence_gguf* g, const char* key, uint32_t* type) {
    if (!g || !key || !type) return FENCE_ERROR_INVALID_VALUE;
    const GGUFMetadataKV* kv = g->file.find_metadata(key);
    if (!kv) return FENCE_ERROR_NOT_FOUND;
    *type = static_cast<uint32_t>(kv->type);
    return FENCE_SUCCESS;
}

extern "C" int fence_gguf_get_u32(const fence_gguf* g, const char* key, uint32_t* out) {
    return get_typed(g, key, out, GGUFValueType::UINT32, [](const GGUFMetadataValue& v) { return std::get<uint32_t>(v); });
}
extern "C" int fence_gguf_get_i32(const fence_gguf* g, const char* key, int32_t* out) {
    return get_typed(g, key, out, GGUFValueType::INT32, [](const GGUFMetadataValue& v) { return std::get<int32_t>(v); });
}
extern "C" int fence_gguf_get_u64(const fence_gguf* g, const char* key, uint64_t* out) {
    return get_typed(g, key, out, GGUFValueType::UINT64, [](const GGUFMetadataValue& v) { return std::get<uint64_t>(v); });
}
extern "C" int fence_gguf_get_f32(const fence_gguf* g, const char* key, float* out) {
    return get_typed(g, key, out, GGUFValueType::FLOAT32, [](const GGUFMetadataValue& v) { return std::get<float>(v); });
}
extern "C" int fence_gguf_get_bool(const fence_gguf* g, const char* key, int* out) {
    return get_typed(g, key, out, GGUFValueType::BOOL, [](const GGUFMetadataValue& v) { return std::get<bool>(v) ? 1 : 0; });
}
extern "C" int fence_gguf_get_string(const fence_gguf* g, const char* key, const char** out) {
    return get_typed(g, key, out, GGUFValueType::STRING,
                     [](const GGUFMetadataValue& v) { return std::get<std::string>(v).c_str(); });
}
