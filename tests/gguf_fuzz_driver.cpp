// Mutation driver for the GGUF reader, built by tests/test_gguf_cpu.py with
// the host sanitizers (address, undefined): parses `n` seeded mutants of the
// image in argv[1] and touches every byte range the reader hands out.  Exit
// status 0 when every mutant parsed or was rejected cleanly.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "rrr_gguf.h"

namespace rrr {
int set_error(int code, const char *) { return code; }
}  // namespace rrr

static unsigned touch(const void *p, uint64_t n)
{
    if (!n) return 0;
    const unsigned char *c = (const unsigned char *)p;
    return c[0] + c[n - 1];
}

int main(int argc, char **argv)
{
    if (argc != 4) return 2;
    FILE *f = fopen(argv[1], "rb");
    if (!f) return 2;
    std::vector<unsigned char> img;
    for (int ch; (ch = fgetc(f)) != EOF;) img.push_back((unsigned char)ch);
    fclose(f);
    const long n = atol(argv[2]);
    std::mt19937_64 rng(strtoull(argv[3], nullptr, 10));
    unsigned sink = 0;
    long accepted = 0;
    for (long it = 0; it < n; ++it) {
        std::vector<unsigned char> m = img;
        const int kind = (int)(rng() % 4);
        if (kind == 0) {                      // random byte overwrites
            for (int k = 1 + (int)(rng() % 8); k > 0; --k) m[rng() % m.size()] = (unsigned char)rng();
        } else if (kind == 1) {               // truncation
            m.resize(rng() % m.size());
        } else if (kind == 2) {               // one 8-byte field set to an extreme value
            const size_t at = rng() % (m.size() > 8 ? m.size() - 8 : 1);
            const uint64_t vals[] = {0, 1, 0xFFFFFFFFull, 0x7FFFFFFFFFFFFFFFull, ~0ull, 1ull << 40};
            const uint64_t v = vals[rng() % 6];
            if (m.size() >= at + 8) memcpy(&m[at], &v, 8);
        } else {                              // bit flips in the header
            for (int k = 1 + (int)(rng() % 4); k > 0; --k) {
                const size_t at = rng() % (m.size() < 512 ? m.size() : 512);
                m[at] ^= (unsigned char)(1u << (rng() % 8));
            }
        }
        // an exact-size heap copy, so that any read past the image is caught
        unsigned char *buf = (unsigned char *)malloc(m.size() ? m.size() : 1);
        if (!m.empty()) memcpy(buf, m.data(), m.size());
        rrr_gguf *g = nullptr;
        const int rc = rrr_gguf_open_memory(buf, m.size(), &g);
        if (rc == RRR_OK) {
            ++accepted;
            uint64_t nt = 0, nkv = 0;
            rrr_gguf_header(g, nullptr, &nt, &nkv, nullptr, nullptr);
            for (uint64_t i = 0; i < nkv; ++i) {
                rrr_gguf_kv kv;
                if (rrr_gguf_kv_at(g, i, &kv) != RRR_OK) return 3;
                sink += touch(kv.key, kv.key_len) + touch(kv.data, kv.bytes);
                if (kv.type == RRR_GGUF_STRING || (kv.type == RRR_GGUF_ARRAY && kv.elem_type == RRR_GGUF_STRING)) {
                    const uint64_t cnt = kv.type == RRR_GGUF_STRING ? 1 : kv.count;
                    for (uint64_t s = 0; s < cnt; ++s) {
                        const char *p;
                        uint64_t len;
                        if (rrr_gguf_kv_strings(g, i, s, 1, &p, &len) != RRR_OK) return 4;
                        sink += touch(p, len);
                    }
                }
                uint64_t u;
                double d;
                rrr_gguf_get_u64(g, kv.key, &u);
                rrr_gguf_get_f64(g, kv.key, &d);
            }
            for (uint64_t i = 0; i < nt; ++i) {
                rrr_gguf_tensor t;
                if (rrr_gguf_tensor_at(g, i, &t) != RRR_OK) return 5;
                sink += touch(t.name, t.name_len) + touch(t.data, t.bytes);
            }
            if (rrr_gguf_close(g) != RRR_OK) return 6;
        } else if (g != nullptr || rc >= 0) {
            return 7;
        }
        free(buf);
    }
    printf("mutants %ld accepted %ld sink %u\n", n, accepted, sink);
    return 0;
}
