// pools_dump -- test infrastructure only: drives the reference's own C++ chunk transcodes
// (src/open_qwen36/pools.cpp, compiled from /root/reference by oracle/Makefile) so the tests
// can hold this build's oracle (and through it the GPU repacks) to them byte for byte.
//
//   pools_dump OP IN OUT
//
// IN holds whole source chunks; OUT receives the transcoded chunks, in the same order.
//   requant    8704 B q8 chunks   -> 5120 B q4_1 chunks   pools::requant_q4_1_chunks
//   q4k        4736 B Q4_K chunks -> 5120 B q4_1 chunks   pools::q4k_to_q4_1_chunks
//   q4_0       5120 B signed      -> 5120 B q4_1 chunks   pools::q4_0_to_q4_1_chunks
//   split_hi   8704 B q8 chunks   -> 5120 B "hi" chunks   pools::split_q4_1_chunks(hi = true)
//   split_lo   8704 B q8 chunks   -> 5120 B "lo" chunks   pools::split_q4_1_chunks(hi = false)
// Exit status 0 on success; 2 on usage errors; 3 when the reference code throws.
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "open_qwen36/pools.hpp"

namespace {

bool read_all(const char* path, std::vector<uint8_t>& out) {
    FILE* fp = std::fopen(path, "rb");
    if (!fp) return false;
    std::fseek(fp, 0, SEEK_END);
    const long n = std::ftell(fp);
    std::fseek(fp, 0, SEEK_SET);
    out.resize(n > 0 ? (size_t)n : 0);
    const bool ok = n >= 0 && std::fread(out.data(), 1, out.size(), fp) == out.size();
    std::fclose(fp);
    return ok;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 4) {
        std::fprintf(stderr, "usage: %s requant|q4k|q4_0|split_hi|split_lo IN OUT\n", argv[0]);
        return 2;
    }
    const std::string op = argv[1];
    size_t in_chunk = 0;
    if (op == "requant" || op == "split_hi" || op == "split_lo") in_chunk = 8704;
    else if (op == "q4k") in_chunk = 4736;
    else if (op == "q4_0") in_chunk = 5120;
    else {
        std::fprintf(stderr, "unknown op %s\n", op.c_str());
        return 2;
    }
    std::vector<uint8_t> src;
    if (!read_all(argv[2], src) || src.size() % in_chunk != 0) {
        std::fprintf(stderr, "cannot read whole %zu-byte chunks from %s\n", in_chunk, argv[2]);
        return 2;
    }
    const size_t nch = src.size() / in_chunk;
    std::vector<uint8_t> dst(nch * 5120, 0);
    try {
        namespace P = open_qwen36::pools;
        if (op == "requant") P::requant_q4_1_chunks(src.data(), nch, dst.data());
        else if (op == "q4k") P::q4k_to_q4_1_chunks(src.data(), nch, dst.data());
        else if (op == "q4_0") P::q4_0_to_q4_1_chunks(src.data(), nch, dst.data());
        else P::split_q4_1_chunks(src.data(), nch, op == "split_hi", dst.data());
    } catch (const std::exception& e) {
        std::printf("error\t%s\n", e.what());
        return 3;
    }
    FILE* fp = std::fopen(argv[3], "wb");
    if (!fp || std::fwrite(dst.data(), 1, dst.size(), fp) != dst.size()) {
        std::fprintf(stderr, "cannot write %s\n", argv[3]);
        return 1;
    }
    std::fclose(fp);
    return 0;
}
