// Host driver for a sanitizer build of the ZCBLK01 reader
// (wohper_amd/csrc/quant_block.h): mutates a seed block (byte flips in the
// header, records and names; truncations; 64-bit offset fields set to
// values near the end of the block or near 2^64) and runs the header,
// per-record and expert parsers on an exactly sized heap copy, so any read
// outside the block is reported.  Built and run by tests/test_quant_block.py.
//   usage: quant_block_asan SEED_BLOCK ITERATIONS
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "quant_block.h"

namespace {

uint64_t g_state = 0x9e3779b97f4a7c15ull;

uint64_t next() {  // xorshift64*
    g_state ^= g_state >> 12;
    g_state ^= g_state << 25;
    g_state ^= g_state >> 27;
    return g_state * 0x2545f4914f6cdd1dull;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    FILE* f = std::fopen(argv[1], "rb");
    if (!f) return 2;
    std::vector<uint8_t> seed;
    for (int ch; (ch = std::fgetc(f)) != EOF;) seed.push_back((uint8_t)ch);
    std::fclose(f);
    const long iters = std::atol(argv[2]);
    long accepted = 0;
    for (long it = 0; it < iters; ++it) {
        std::vector<uint8_t> b(seed);
        const uint64_t kind = next() % 4;
        if (kind == 0) {
            b.resize(next() % (seed.size() + 1));
        } else if (kind == 1 || kind == 2) {
            const size_t span = std::min<size_t>(b.size(), 40 + 6 * 52 + 240);
            for (uint64_t k = 1 + next() % 3; k-- > 0;) b[next() % span] = (uint8_t)next();
        } else {
            // one 64-bit offset or length field of a record, or of the header
            const size_t n = (b.size() - 40) / 52;
            const size_t rec = 40 + 52 * (next() % (n ? n : 1));
            const size_t fields[] = {24, 32, rec + 12, rec + 20, rec + 28, rec + 36};
            const size_t at = fields[next() % 6];
            const uint64_t picks[] = {b.size() - next() % 16, ~0ull - next() % 64, next() % (b.size() + 64)};
            const uint64_t v = picks[next() % 3];
            if (at + 8 <= b.size()) std::memcpy(b.data() + at, &v, 8);
        }
        // exactly sized heap copy: the sanitizer sees any read past the end
        uint8_t* heap = (uint8_t*)std::malloc(b.size() ? b.size() : 1);
        std::memcpy(heap, b.data(), b.size());
        whqb::Reader r(heap, b.size());
        whqb::Header h;
        whqb::Error err;
        if (whqb::parse_header(r, &h, &err)) {
            for (size_t i = 0; i < h.tensor_count && i < 64; ++i) {
                whqb::Tensor t;
                whqb::Error e2;
                if (whqb::tensor_at(r, h, i, &t, &e2)) {
                    volatile uint8_t sink = 0;
                    for (size_t k = 0; k < t.name_len; ++k) sink ^= heap[t.name_off + k];
                    for (uint32_t d = 0; d < t.rank && d < 8; ++d) sink ^= (uint8_t)t.dim(r, d);
                    if (t.data_len) sink ^= heap[t.data_off] ^ heap[t.data_off + t.data_len - 1];
                }
            }
        }
        whqb::Fp4 p[3];
        whqb::Error e3;
        if (whqb::fp4_expert(heap, b.size(), p, &e3)) {
            ++accepted;
            for (const whqb::Fp4& m : p) {
                volatile uint8_t sink = heap[m.weight_off] ^ heap[m.weight_off + m.weight_len - 1] ^
                                        heap[m.scale_off] ^ heap[m.scale_off + m.scale_len - 1];
                (void)sink;
            }
        } else {
            char text[256];
            whqb::describe(e3, text, sizeof text);
        }
        std::free(heap);
    }
    std::printf("accepted %ld of %ld mutated blocks\n", accepted, iters);
    return 0;
}
