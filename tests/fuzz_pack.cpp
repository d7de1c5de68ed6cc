// Mutation fuzzing of the pack reader (host code), built with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_pack.py: usage fuzz_pack ITERATIONS SEED_PACK...
// Each iteration mutates one of the seed packs (bit flips, bytes set to JSON punctuation or
// extreme numbers, truncation, inserted or dropped bytes, a random index offset or length; half of
// the iterations only inside the JSON index, with the trailer's length kept consistent), opens it
// with tg_pack_from_bytes and, when it is accepted, walks every metadata item and entry and touches
// the first and last byte of each entry's data and scales. A memory error stops the run.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>
#include "../include/telmo_hip.h"

static std::vector<uint8_t> read_file(const char *p) {
    FILE *f = fopen(p, "rb");
    std::vector<uint8_t> v;
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
    if (argc < 3) {
        printf("usage: fuzz_pack ITERATIONS SEED_PACK...\n");
        return 2;
    }
    const long iters = atol(argv[1]);
    std::vector<std::vector<uint8_t>> seeds;
    for (int i = 2; i < argc; i++) {
        seeds.push_back(read_file(argv[i]));
        if (seeds.back().size() < 24) {
            printf("no usable seed %s\n", argv[i]);
            return 1;
        }
    }
    std::mt19937_64 rng(12345);
    const uint8_t interesting[] = {0, 1, 0x7f, 0x80, 0xff, '"', '{', '}', '[', ']', ':', ',', '0', '9', '-', 'e', '.', '\\', ' '};
    long ok = 0, refused = 0;
    for (long it = 0; it < iters; it++) {
        std::vector<uint8_t> d = seeds[rng() % seeds.size()];
        const int muts = 1 + rng() % 8;
        // half the iterations mutate only the JSON index (between its offset and the trailer)
        uint64_t j0 = 0, jl = 0;
        memcpy(&j0, d.data() + d.size() - 24, 8);
        memcpy(&jl, d.data() + d.size() - 16, 8);
        const bool json_only = it % 2 == 1;
        for (int m = 0; m < muts && !d.empty(); m++) {
            size_t at = rng() % d.size();
            if (json_only && jl > 0 && j0 + jl <= d.size()) at = j0 + rng() % jl;
            if (at >= d.size()) at = d.size() - 1;
            switch (rng() % 8) {
            case 0: d[at] ^= (uint8_t)(1u << (rng() % 8)); break;
            case 1: d[at] = interesting[rng() % sizeof interesting]; break;
            case 2: if (!json_only) d.resize(rng() % (d.size() + 1)); break;
            case 3: d.insert(d.begin() + at, interesting[rng() % sizeof interesting]); if (json_only) jl++; break;
            case 4: d.erase(d.begin() + at); if (json_only && jl) jl--; break;
            case 5: {  // the trailer's offset or length
                if (d.size() >= 24) {
                    uint64_t v = rng();
                    if (rng() % 2) v %= d.size() + 64;
                    memcpy(d.data() + d.size() - 24 + 8 * (rng() % 2), &v, 8);
                }
                break;
            }
            case 6: {  // a JSON number somewhere: replace a digit run with a large or negative one
                const char *big[] = {"18446744073709551615", "-1", "1e308", "4294967296", "0", "99999999999999999999999"};
                const char *s = big[rng() % 6];
                d.insert(d.begin() + at, s, s + strlen(s));
                if (json_only) jl += strlen(s);
                break;
            }
            default: d[at] = (uint8_t)rng(); break;
            }
        }
        // keep the trailer's index length consistent with the mutated index
        if (json_only && d.size() >= 24 && (rng() % 4) != 0) memcpy(d.data() + d.size() - 16, &jl, 8);
        tg_pack *p = nullptr;
        if (tg_pack_from_bytes(d.data(), d.size(), &p) == TG_OK && p) {
            ok++;
            (void)tg_pack_model(p);
            const size_t nm = tg_pack_meta_count(p);
            for (size_t i = 0; i < nm; i++) {
                const char *k = nullptr, *v = nullptr;
                if (tg_pack_meta_at(p, i, &k, &v) == TG_OK && k) (void)tg_pack_meta(p, k);
            }
            const size_t ne = tg_pack_entry_count(p);
            for (size_t i = 0; i < ne; i++) {
                tg_pack_entry e;
                if (tg_pack_entry_at(p, i, &e) == TG_OK) {
                    tg_pack_entry f;
                    (void)tg_pack_find(p, e.name, &f);
                    // touch the entry's bytes: they must lie inside the buffer
                    volatile uint8_t sink = 0;
                    const uint8_t *b = static_cast<const uint8_t *>(e.data);
                    if (e.bytes) sink ^= b[0] ^ b[e.bytes - 1];
                    if (e.scales && e.n_scales) sink ^= (uint8_t)(e.scales[0] + e.scales[e.n_scales - 1]);
                    (void)sink;
                }
            }
            tg_pack_close(p);
        } else {
            refused++;
            (void)tg_pack_last_error();
        }
    }
    printf("iterations %ld: parsed %ld, refused %ld\n", iters, ok, refused);
    return 0;
}
