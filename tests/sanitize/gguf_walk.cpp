// gguf_walk.cpp -- test harness: opens each GGUF file named on the command
// line through the C ABI (include/fence/gguf.h) and reads everything the
// reader exposes: every tensor's info and the first and last byte of its
// data, the keys a Qwen3 load queries, and keys that are absent.  Built with
// AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_gguf_sanitized.py,
// so any out-of-bounds read, use after free or overflow in the reader aborts.
// Prints "opened <n> rejected <m>"; exit status 1 if a rejected file's status
// is not FENCE_ERROR_BAD_FILE or an opened file's tensor lies outside it.
#include <cstdint>
#include <cstdio>

#include "fence/gguf.h"

int main(int argc, char** argv) {
    const char* keys[] = {"general.architecture", "general.alignment", "qwen3.block_count",
                          "qwen3.embedding_length", "qwen3.attention.head_count",
                          "qwen3.attention.layer_norm_rms_epsilon", "qwen3.rope.freq_base",
                          "tok", "f", "n", "", "no.such.key"};
    int opened = 0, rejected = 0, bad = 0;
    unsigned sink = 0;
    for (int a = 1; a < argc; ++a) {
        fence_gguf* g = nullptr;
        char err[256];
        const int st = fence_gguf_open(argv[a], &g, err, sizeof err);
        if (st != FENCE_SUCCESS) {
            ++rejected;
            if (st != FENCE_ERROR_BAD_FILE) {
                std::printf("%s: status %d (%s)\n", argv[a], st, err);
                bad = 1;
            }
            continue;
        }
        ++opened;
        const uint64_t n = fence_gguf_tensor_count(g);
        const uint64_t size = fence_gguf_file_size(g), data0 = fence_gguf_data_offset(g);
        sink += fence_gguf_version(g) + static_cast<unsigned>(fence_gguf_metadata_count(g));
        for (uint64_t i = 0; i < n; ++i) {
            fence_gguf_tensor_info t;
            if (fence_gguf_tensor_at(g, i, &t) != FENCE_SUCCESS) {
                bad = 1;
                continue;
            }
            fence_gguf_tensor_info u;
            sink += static_cast<unsigned>(fence_gguf_find_tensor(g, t.name, &u));
            if (t.n_dims > 4 || data0 + t.offset + t.data_size_bytes > size) {
                std::printf("%s: tensor %llu outside the file\n", argv[a], static_cast<unsigned long long>(i));
                bad = 1;
            }
            for (uint32_t d = 0; d < t.n_dims; ++d) sink += static_cast<unsigned>(t.dims[d]);
            if (t.data_size_bytes) {
                const unsigned char* p = static_cast<const unsigned char*>(t.data);
                sink += p[0] + p[t.data_size_bytes - 1];
            }
        }
        for (const char* k : keys) {
            uint32_t ty = 0, u32 = 0;
            int32_t i32 = 0;
            uint64_t u64 = 0;
            float f = 0;
            int b = 0;
            const char* s = nullptr;
            sink += static_cast<unsigned>(fence_gguf_metadata_type(g, k, &ty));
            sink += static_cast<unsigned>(fence_gguf_get_u32(g, k, &u32) + fence_gguf_get_i32(g, k, &i32) +
                                          fence_gguf_get_u64(g, k, &u64) + fence_gguf_get_f32(g, k, &f) +
                                          fence_gguf_get_bool(g, k, &b));
            if (fence_gguf_get_string(g, k, &s) == FENCE_SUCCESS && s)
                for (const char* c = s; *c; ++c) sink += static_cast<unsigned char>(*c);
        }
        fence_gguf_close(g);
    }
    std::printf("opened %d rejected %d (%u)\n", opened, rejected, sink & 1u);
    return bad;
}
