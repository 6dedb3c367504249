// Opens each GGUF file named on the command line with the library's reader
// and reads everything it exposes: the header, every tensor record (and the
// first and last byte of its data), every metadata entry with its raw bytes,
// the scalar lookups and the Llama configuration.  Files the reader rejects
// are skipped.  Built with AddressSanitizer and UBSan over host/gguf.cpp, it
// shows that hostile files are read without out-of-bounds accesses or
// undefined behaviour.  Prints "OK <opened> <rejected>".
#include <cstdio>
#include <cstring>

#include "ulspec.h"

int main(int argc, char** argv)
{
    int opened = 0, rejected = 0;
    unsigned sink = 0;
    for (int a = 1; a < argc; ++a) {
        ulspec_gguf* g = nullptr;
        char err[256];
        if (ulspec_gguf_open(argv[a], &g, err, sizeof(err)) != ULSPEC_OK) {
            ++rejected;
            continue;
        }
        ++opened;
        uint32_t version = 0;
        uint64_t n_t = 0, n_kv = 0, align = 0, data_off = 0;
        ulspec_gguf_header(g, &version, &n_t, &n_kv, &align, &data_off);
        for (uint64_t i = 0; i < n_t; ++i) {
            const char* name = nullptr;
            uint32_t type = 0, nd = 0;
            uint64_t ne[4], off = 0, nb = 0;
            const void* data = nullptr;
            if (ulspec_gguf_tensor(g, i, &name, &type, &nd, ne, &off, &nb, &data) != ULSPEC_OK) continue;
            sink += (unsigned)std::strlen(name);
            if (data && nb) sink += ((const unsigned char*)data)[0] + ((const unsigned char*)data)[nb - 1];
            uint64_t idx = 0;
            ulspec_gguf_find_tensor(g, name, &idx);
        }
        for (uint64_t i = 0; i < n_kv; ++i) {
            const char* key = nullptr;
            uint32_t vt = 0, at = 0;
            uint64_t n = 0;
            if (ulspec_gguf_kv(g, i, &key, &vt, &at, &n) != ULSPEC_OK) continue;
            const void* data = nullptr;
            uint64_t nb = 0;
            if (ulspec_gguf_kv_bytes(g, i, &data, &nb) == ULSPEC_OK && nb)
                sink += ((const unsigned char*)data)[0] + ((const unsigned char*)data)[nb - 1];
            int64_t iv;
            double fv;
            const char* sv;
            uint64_t sl;
            ulspec_gguf_get_int(g, key, &iv);
            ulspec_gguf_get_float(g, key, &fv);
            if (ulspec_gguf_get_str(g, key, &sv, &sl) == ULSPEC_OK && sl) sink += (unsigned char)sv[sl - 1];
        }
        ulspec_model_cfg cfg;
        ulspec_gguf_llama_cfg(g, 0, &cfg);
        ulspec_gguf_close(g);
    }
    std::printf("OK %d %d %u\n", opened, rejected, sink & 1u);
    return 0;
}
