// gguf_dump -- test infrastructure only: drives the reference's own C++ GGUF reader
// (src/gguf/gguf_file.cpp, compiled from /root/reference by oracle/Makefile) so the tests
// can hold this build's GGUF parser and Q4_K law to it.
//
//   gguf_dump FILE OUTDIR [KEY ...]
//
// stdout, one record per line, tab-separated:
//   kv      KEY   VALUE            (the reader's string view of each KEY asked for)
//   tensor  IDX   NAME  TYPE  DIMS(fastest-first, comma-joined)  OFFSET
// and OUTDIR/IDX.f32 holds GgufFile::f32_all(NAME) (the reader's own dequant), raw f32.
#include <cstdio>
#include <exception>
#include <string>

#include "gguf/gguf_file.hpp"

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s FILE OUTDIR [KEY ...]\n", argv[0]);
        return 2;
    }
    try {
        open_qwen36::GgufFile f(argv[1]);
        for (int a = 3; a < argc; ++a)
            std::printf("kv\t%s\t%s\n", argv[a], f.kv_has(argv[a]) ? f.kv_str(argv[a]).c_str() : "<absent>");
        int idx = 0;
        for (const std::string& name : f.tensor_names()) {
            const auto& t = f.tensor(name);
            std::string dims;
            for (size_t i = 0; i < t.dims.size(); ++i) dims += (i ? "," : "") + std::to_string(t.dims[i]);
            std::printf("tensor\t%d\t%s\t%s\t%s\t%llu\n", idx, name.c_str(),
                        open_qwen36::GgufFile::type_name(t.type), dims.c_str(),
                        (unsigned long long)t.offset);
            const std::vector<float> v = f.f32_all(name);
            const std::string out = std::string(argv[2]) + "/" + std::to_string(idx) + ".f32";
            FILE* fp = std::fopen(out.c_str(), "wb");
            if (!fp || std::fwrite(v.data(), sizeof(float), v.size(), fp) != v.size()) {
                std::fprintf(stderr, "cannot write %s\n", out.c_str());
                return 1;
            }
            std::fclose(fp);
            ++idx;
        }
    } catch (const std::exception& e) {
        std::printf("error\t%s\n", e.what());
        return 3;
    }
    return 0;
}
