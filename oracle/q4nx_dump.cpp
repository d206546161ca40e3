// q4nx_dump -- test infrastructure only: drives the reference's own C++ .q4nx reader
// (src/open_qwen36/q4nx_file.cpp, compiled from /root/reference by oracle/Makefile) so the
// tests can hold this build's container parser to it.
//
//   q4nx_dump FILE OUTDIR [--meta KEY]... NAME...
//
// stdout, tab-separated: "count N" (tensors the header lists); "meta KEY VALUE" per --meta;
// per NAME "tensor IDX NAME DTYPE SHAPE(comma-joined) START END CHUNK_BYTES"; and
// OUTDIR/IDX.bin holds the tensor's raw bytes (Q4nxFile::raw), OUTDIR/IDX.f32 its
// Q4nxFile::bf16() / f32() decode for BF16 / F32 tensors.
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "open_qwen36/q4nx_file.hpp"

static bool write_file(const std::string& path, const void* p, size_t n) {
    FILE* fp = std::fopen(path.c_str(), "wb");
    if (!fp) return false;
    const bool ok = std::fwrite(p, 1, n, fp) == n;
    std::fclose(fp);
    return ok;
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s FILE OUTDIR [--meta KEY]... NAME...\n", argv[0]);
        return 2;
    }
    try {
        open_qwen36::Q4nxFile f(argv[1]);
        const std::string out = argv[2];
        std::printf("count\t%zu\n", f.tensor_count());
        int idx = 0;
        for (int a = 3; a < argc; ++a) {
            if (!std::strcmp(argv[a], "--meta") && a + 1 < argc) {
                std::printf("meta\t%s\t%s\n", argv[a + 1], f.metadata(argv[a + 1]).c_str());
                ++a;
                continue;
            }
            const std::string name = argv[a];
            const auto& m = f.meta(name);
            std::string shape;
            for (size_t i = 0; i < m.shape.size(); ++i) shape += (i ? "," : "") + std::to_string(m.shape[i]);
            std::printf("tensor\t%d\t%s\t%s\t%s\t%zu\t%zu\t%zu\n", idx, name.c_str(), m.dtype.c_str(), shape.c_str(),
                        m.start, m.end, f.chunk_bytes(name));
            size_t nb = 0;
            const uint8_t* p = f.raw(name, &nb);
            if (!write_file(out + "/" + std::to_string(idx) + ".bin", p, nb)) return 1;
            if (m.dtype == "BF16" || m.dtype == "F32") {
                const std::vector<float> v = m.dtype == "BF16" ? f.bf16(name) : f.f32(name);
                if (!write_file(out + "/" + std::to_string(idx) + ".f32", v.data(), v.size() * 4)) return 1;
            }
            ++idx;
        }
    } catch (const std::exception& e) {
        std::printf("error\t%s\n", e.what());
        return 3;
    }
    return 0;
}
