/*
 * fence/gguf.h -- C ABI of the GGUF reader (include/fence/gguf_parser.hpp),
 * for hosts that cannot use the C++ class (ctypes, cgo, JNI).  Each entry
 * point replaces a member of the reference's GGUFFile
 * (src/gguf/gguf_parser.h:130-217); the file stays memory-mapped until
 * fence_gguf_close, and every pointer handed out (names, strings, tensor
 * data) is valid until then.
 *
 * Statuses: FENCE_SUCCESS, FENCE_ERROR_INVALID_VALUE (null argument),
 * FENCE_ERROR_NOT_FOUND, FENCE_ERROR_TYPE_MISMATCH (the reference's get_*
 * throw std::runtime_error for both), FENCE_ERROR_BAD_FILE (open failed; the
 * reason is copied into err), FENCE_ERROR_OUT_OF_MEMORY.
 */
#ifndef FENCE_GGUF_H
#define FENCE_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "fence/ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fence_gguf fence_gguf;

/* GGUFTensorInfo, src/gguf/gguf_parser.h:93-108 (type: the GGUF type number). */
typedef struct {
    const char* name;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t type;
    uint64_t offset;
    const void* data;
    uint64_t data_size_bytes;
} fence_gguf_tensor_info;

/* GGUFFile::open, src/gguf/gguf_parser.h:146.  err (may be NULL) receives the
 * reason of a failure, truncated to err_len bytes. */
int fence_gguf_open(const char* path, fence_gguf** out, char* err, size_t err_len);
/* GGUFFile::close (and the destructor), src/gguf/gguf_parser.h:149. */
void fence_gguf_close(fence_gguf* g);

/* version(), tensor_count(), metadata_count(), file_size(), data_offset(),
 * src/gguf/gguf_parser.h:155-157,183-186; alignment in effect. */
uint32_t fence_gguf_version(const fence_gguf* g);
uint64_t fence_gguf_tensor_count(const fence_gguf* g);
uint64_t fence_gguf_metadata_count(const fence_gguf* g);
uint64_t fence_gguf_file_size(const fence_gguf* g);
uint64_t fence_gguf_data_offset(const fence_gguf* g);
uint32_t fence_gguf_alignment(const fence_gguf* g);

/* find_tensor, src/gguf/gguf_parser.h:177; tensors()[index], :174. */
int fence_gguf_find_tensor(const fence_gguf* g, const char* name, fence_gguf_tensor_info* out);
int fence_gguf_tensor_at(const fence_gguf* g, uint64_t index, fence_gguf_tensor_info* out);

/* find_metadata(key)->type, src/gguf/gguf_parser.h:163 (array keys are not
 * stored: NOT_FOUND). */
int fence_gguf_metadata_type(const fence_gguf* g, const char* key, uint32_t* type);
/* get_u32 / get_i32 / get_u64 / get_f32 / get_bool / get_string,
 * src/gguf/gguf_parser.h:166-171. */
int fence_gguf_get_u32(const fence_gguf* g, const char* key, uint32_t* out);
int fence_gguf_get_i32(const fence_gguf* g, const char* key, int32_t* out);
int fence_gguf_get_u64(const fence_gguf* g, const char* key, uint64_t* out);
int fence_gguf_get_f32(const fence_gguf* g, const char* key, float* out);
int fence_gguf_get_bool(const fence_gguf* g, const char* key, int* out);
int fence_gguf_get_string(const fence_gguf* g, const char* key, const char** out);

#ifdef __cplusplus
}
#endif

#endif /* FENCE_GGUF_H */
