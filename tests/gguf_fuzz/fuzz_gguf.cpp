// Mutation fuzzing of the GGUF reader under AddressSanitizer (host only).
// usage: fuzz_gguf ITERS SEED_FILE...
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "chat_wgpu.h"

static std::vector<uint8_t> read_file(const char *p) {
    std::vector<uint8_t> v;
    FILE *f = fopen(p, "rb");
    if (!f) return v;
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    v.resize(n);
    if (fread(v.data(), 1, n, f) != (size_t)n) v.clear();
    fclose(f);
    return v;
}

int main(int argc, char **argv) {
    if (argc < 3) return 2;
    const long iters = atol(argv[1]);
    std::vector<std::vector<uint8_t>> seeds;
    for (int i = 2; i < argc; ++i) seeds.push_back(read_file(argv[i]));
    std::mt19937_64 rng(getenv("FUZZ_SEED") ? strtoull(getenv("FUZZ_SEED"), nullptr, 10) : 1234);
    long parsed = 0, tensors_ok = 0, tensors_err = 0;
    const uint64_t interesting[] = {0,           1,          0x7f,       0x80,       0xff,
                                    0x7fff,      0xffff,     0x7fffffff, 0xffffffff, 0x100000000ull,
                                    ~0ull,       ~0ull >> 1, 32,         4096,       65536};
    for (long it = 0; it < iters; ++it) {
        std::vector<uint8_t> b = seeds[rng() % seeds.size()];
        const int nmut = 1 + (int)(rng() % 8);
        for (int k = 0; k < nmut && !b.empty(); ++k) {
            const int op = (int)(rng() % 6);
            const size_t pos = rng() % b.size();
            if (op == 0) {
                b[pos] ^= (uint8_t)(1u << (rng() % 8));
            } else if (op == 1) {
                b[pos] = (uint8_t)rng();
            } else if (op == 2) {  // an interesting little-endian integer of 1/2/4/8 bytes
                const int w = 1 << (rng() % 4);
                const uint64_t v = interesting[rng() % (sizeof interesting / sizeof interesting[0])];
                for (int j = 0; j < w && pos + j < b.size(); ++j) b[pos + j] = (uint8_t)(v >> (8 * j));
            } else if (op == 3) {
                b.resize(pos);
            } else if (op == 4) {  // duplicate a chunk
                const size_t n = 1 + rng() % 32;
                std::vector<uint8_t> c(b.begin() + pos, b.begin() + std::min(b.size(), pos + n));
                b.insert(b.begin() + pos, c.begin(), c.end());
            } else {  // delete a chunk
                const size_t n = 1 + rng() % 32;
                b.erase(b.begin() + pos, b.begin() + std::min(b.size(), pos + n));
            }
        }
        cw_gguf *g = nullptr;
        if (cw_gguf_parse(b.data(), b.size(), &g) != CW_OK) continue;
        ++parsed;
        uint32_t ver = 0;
        uint64_t nt = 0, nm = 0, off = 0;
        cw_gguf_info(g, &ver, &nt, &nm, &off);
        uint32_t u = 0;
        float f = 0;
        char sb[64];
        size_t sl = 0;
        cw_gguf_meta_u32(g, "qwen3.block_count", &u);
        cw_gguf_meta_u32(g, "a.u64", &u);
        cw_gguf_meta_f32(g, "a.f64", &f);
        cw_gguf_meta_f32(g, "qwen3.rope.freq_base", &f);
        cw_gguf_meta_str(g, "general.name", sb, sizeof sb, &sl);
        cw_gguf_meta_str(g, "a.nest", sb, sizeof sb, &sl);
        cw_model_config cfg;
        cw_gguf_model_config(g, 64, CW_F32, &cfg);
        for (uint64_t t = 0; t < nt && t < 64; ++t) {
            char name[256];
            if (cw_gguf_tensor_name(g, t, name, sizeof name) != CW_OK) continue;
            uint32_t dt = 0;
            int nd = 0;
            uint64_t dims[8], ne = 0, toff = 0;
            if (cw_gguf_tensor_info(g, name, &dt, &nd, dims, 8, &ne, &toff) != CW_OK) continue;
            if (ne == 0 || ne > (1u << 22)) continue;
            std::vector<float> out(ne);
            if (cw_gguf_tensor_f32(g, name, out.data(), out.size()) == CW_OK) ++tensors_ok;
            else ++tensors_err;
            if (nd == 2 && dims[0] % 32 == 0 && dims[0] > 0 && dims[1] > 0 &&
                dims[0] * dims[1] <= (1u << 22)) {
                const size_t in_f = dims[0], out_f = dims[1];
                std::vector<uint16_t> sc(out_f * in_f / 32);
                std::vector<uint8_t> q(out_f * in_f / 2);
                cw_gguf_tensor_q4(g, name, out_f, in_f, sc.data(), q.data());
            }
        }
        cw_gguf_close(g);
    }
    printf("iterations %ld, parsed %ld, tensors decoded %ld, refused %ld\n", iters, parsed,
           tensors_ok, tensors_err);
    return 0;
}
