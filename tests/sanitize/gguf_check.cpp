// Host-side GGUF reader, config and Q8 packing of the product (hobbylm_amd/csrc/hg_gguf.cpp)
// driven over valid and malformed files; built with AddressSanitizer and UndefinedBehavior-
// Sanitizer by tests/test_sanitizers.py.  Prints one line per file: the open / config / load
// return codes (errors are expected for malformed files; the sanitizers must stay silent).
#include <stdio.h>

#include <string>
#include <vector>

#include "../../hobbylm_amd/csrc/hg_gguf.h"

int main(int argc, char **argv) {
    for (int a = 1; a < argc; ++a) {
        hg::Gguf g;
        std::string err;
        int rc = g.open(argv[a], err);
        int crc = 1, lrc = 0;
        size_t loaded = 0;
        if (rc == 0) {
            hg_config c{};
            crc = hg::config_from_gguf(g, c, err);
            for (const auto &kv : g.tensors()) {   // every tensor through Gguf::load and, when 2-D, the Q8 packing
                std::vector<float> w;
                const int r = g.load(kv.first, w, err);
                if (r) {
                    lrc = r;
                    continue;
                }
                loaded += w.size();
                const auto &t = kv.second;
                if (t.ne.size() == 2 && t.ne[0] % 32 == 0) {
                    hg::PackedQ8 p;
                    hg::pack_q8_from_f32(w.data(), (uint32_t)t.ne[1], (uint32_t)t.ne[0], p);
                    p.set_scale_storage(!p.f16_exact);
                }
            }
        }
        printf("%s open %d config %d load %d floats %zu %s\n", argv[a], rc, crc, lrc, loaded, err.c_str());
    }
    return 0;
}
