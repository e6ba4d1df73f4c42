// Seeded fuzzer of the library's host code, built with AddressSanitizer + UndefinedBehaviorSanitizer
// by tests/test_sanitizers.py (g++ on the library's own host sources: kk_ckpt.hip, kk_host.cpp):
//   - the torch.save reader (read_model_checkpoint_bytes / read_voice_pack_bytes, what
//     kk_checkpoint_open and kk_voice_load run) on mutations of the corpus files given on the command
//     line: bit flips, byte and 32-bit-field overwrites with boundary values, truncations, inserted
//     and deleted ranges, mutations aimed at the pickle stream; every mutant must be read or refused
//     with std::runtime_error, nothing else;
//   - the ids-level item checks (ids_item_error) and the layout and duration rules (kk_layout_*,
//     kk_durations_from_logits) on random and adversarial arguments, each result checked against
//     the rule it implements.
// Any sanitizer report aborts the run (-fno-sanitize-recover=all); the last line is
// "mutants M read R refused F other 0; host rules N ok".
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "kk_ckpt.h"
#include "kk_host.h"

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t next() {  // splitmix64 (a published generator), a deterministic stream
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
size_t below(size_t n) { return n ? (size_t)(next() % n) : 0; }

std::vector<uint8_t> read_all(const char* path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

// Offsets of the pickle streams (PROTO 2 opcode) in an archive, to aim some mutations there.
std::vector<size_t> pickle_spans(const std::vector<uint8_t>& b) {
    std::vector<size_t> r;
    for (size_t i = 0; i + 1 < b.size(); i++)
        if (b[i] == 0x80 && b[i + 1] == 0x02) r.push_back(i);
    return r;
}

std::vector<uint8_t> mutate(const std::vector<uint8_t>& src, const std::vector<size_t>& pk) {
    std::vector<uint8_t> m = src;
    const int rounds = 1 + (int)below(4);
    for (int k = 0; k < rounds && !m.empty(); k++) {
        // position: anywhere, or within 256 bytes after a pickle stream's start
        size_t at = below(m.size());
        if (!pk.empty() && below(2)) at = std::min(m.size() - 1, pk[below(pk.size())] + below(256));
        switch (below(7)) {
            case 0:  // bit flips
                for (int i = 0, n = 1 + (int)below(8); i < n; i++) m[below(m.size())] ^= (uint8_t)(1u << below(8));
                break;
            case 1: {  // bytes to boundary values
                static const uint8_t v[] = {0x00, 0x01, 0x7f, 0x80, 0xff, 'K', 'J', 0x8a, 0x85, 'R', '.', 'c'};
                for (int i = 0, n = 1 + (int)below(4); i < n && at + i < m.size(); i++) m[at + i] = v[below(sizeof v)];
                break;
            }
            case 2: {  // a 32-bit little-endian field to a boundary value
                static const uint32_t v[] = {0u, 1u, 2u, 0x7fffffffu, 0x80000000u, 0xffffffffu, 0xfffffffeu, 4096u};
                const uint32_t x = v[below(8)];
                for (int i = 0; i < 4 && at + i < m.size(); i++) m[at + i] = (uint8_t)(x >> (8 * i));
                break;
            }
            case 3:  // truncation
                m.resize(below(m.size() + 1));
                break;
            case 4: {  // insertion of random bytes
                std::vector<uint8_t> ins(1 + below(16));
                for (auto& c : ins) c = (uint8_t)next();
                m.insert(m.begin() + (long)at, ins.begin(), ins.end());
                break;
            }
            case 5: {  // deletion of a range
                const size_t n = std::min(m.size() - at, 1 + below(16));
                m.erase(m.begin() + (long)at, m.begin() + (long)(at + n));
                break;
            }
            default:  // random byte
                m[at] = (uint8_t)next();
        }
    }
    return m;
}

long g_host_ok = 0;
void require(bool ok, const char* what) {
    if (!ok) {
        std::fprintf(stderr, "host rule violated: %s\n", what);
        std::fflush(stderr);
        std::abort();
    }
    g_host_ok++;
}

void fuzz_host_rules(int iters) {
    for (int it = 0; it < iters; it++) {
        // ids-level item checks on random fields
        std::vector<int64_t> ids(1 + below(600));
        for (auto& x : ids) x = below(8) ? (int64_t)below(178) : (int64_t)(next() % 1000) - 500;
        float ref_s[256] = {0.f};
        kk_item item{};
        item.ids = below(16) ? ids.data() : nullptr;
        item.n_ids = below(8) ? (int32_t)ids.size() : (int32_t)(next() % 2000) - 1000;
        if (item.n_ids > (int32_t)ids.size()) item.n_ids = (int32_t)ids.size();  // the caller's array bound
        item.ref_s = below(16) ? ref_s : nullptr;
        const float speeds[] = {1.f, 0.5f, 0.f, -1.f, std::numeric_limits<float>::infinity(), std::nanf(""), 1e-30f};
        item.speed = speeds[below(7)];
        item.noise_kind = (int32_t)below(4) - 1;
        const std::string e = kk::ids_item_error(item, it);
        bool want_ok = item.ids && item.ref_s && item.n_ids >= 2 && item.n_ids <= 512 && std::isfinite(item.speed) &&
                       item.speed > 0.f && (item.noise_kind == KK_NOISE_COUNTER || item.noise_kind == KK_NOISE_FIXED);
        if (want_ok)
            for (int i = 0; i < item.n_ids; i++) want_ok = want_ok && ids[i] >= 0 && ids[i] < 178;
        require(e.empty() == want_ok, "ids_item_error");

        // frame layout: a[b] = sum of (N_j + 2), refusals of negative counts
        const int nb = 1 + (int)below(40);
        std::vector<int64_t> nf(nb), a(nb);
        for (auto& x : nf) x = below(20) ? (int64_t)below(900) : -(int64_t)below(5) - 1;
        const int64_t ln = kk_layout_frames(nf.data(), nb, a.data());
        bool neg = false;
        for (auto x : nf) neg = neg || x < 0;
        require(neg ? ln == KK_ERR_INVALID : ln >= 0, "kk_layout_frames refusal");
        if (neg) continue;
        int64_t acc = 0;
        for (int b = 0; b < nb; b++) {
            require(a[b] == acc, "kk_layout_frames start");
            acc += nf[b] + kk::kGapN;
        }
        require(ln == acc, "kk_layout_frames width");
        // col_item over the domain, with a planted overlap or overrun now and then
        std::vector<int64_t> st(a), le(nf);
        const int plant = (int)below(6);
        if (plant == 0 && nb > 1) st[1] = st[0];                  // overlap (when both are non-empty)
        if (plant == 1) le[nb - 1] = ln - st[nb - 1] + 1;         // past the domain
        if (plant == 2) st[0] = -1;                               // negative start
        if (plant == 3) le[0] = std::numeric_limits<int64_t>::max();  // would wrap start + len
        std::vector<int32_t> ci((size_t)ln + 1);
        const int rc = kk_layout_col_item(ln, st.data(), le.data(), nb, ci.data());
        bool overlap = plant == 0 && nb > 1 && le[0] > 0 && le[1] > 0;
        bool want_bad = overlap || plant == 1 || plant == 2 || (plant == 3 && ln >= 0);
        if (plant == 3 && le[0] <= ln - st[0]) want_bad = false;
        require(want_bad ? rc == KK_ERR_INVALID : rc == KK_OK, "kk_layout_col_item refusal");
        if (rc == KK_OK)
            for (int b = 0; b < nb; b++)
                for (int64_t t = st[b]; t < st[b] + le[b]; t++) require(ci[(size_t)t] == b, "kk_layout_col_item owner");
        // src_row: every frame of item b names its token row; durations that overrun the domain
        // and negative starts are refused
        std::vector<std::vector<int64_t>> dur(nb);
        std::vector<const int64_t*> dp(nb);
        std::vector<int32_t> nt(nb);
        std::vector<int64_t> ts(nb), aa(a);
        int64_t rows = 0;
        for (int b = 0; b < nb; b++) {
            nt[b] = (int32_t)below(12);
            dur[b].assign((size_t)nt[b], 0);
            int64_t left = nf[b];
            for (int t = 0; t < nt[b]; t++) {
                const int64_t d = t + 1 == nt[b] ? left : (int64_t)below((size_t)left + 1);
                dur[b][(size_t)t] = d, left -= d;
            }
            if (nt[b] == 0 && nf[b] > 0) nt[b] = 0;
            dp[b] = dur[b].data();
            ts[b] = rows, rows += nt[b] + kk::kGapT;
        }
        const int sp = (int)below(5);
        if (sp == 0 && nt[nb - 1] > 0) dur[nb - 1][0] += 3;  // overruns the domain
        if (sp == 1) aa[0] = -(int64_t)below(4) - 1;          // negative start
        std::vector<int32_t> sr((size_t)ln + 1);
        const int rs = kk_layout_src_row(dp.data(), nt.data(), nb, ts.data(), aa.data(), ln, sr.data());
        if (sp == 1) require(rs == KK_ERR_INVALID, "kk_layout_src_row negative start");
        if (rs == KK_OK && sp > 1) {
            for (int b = 0; b < nb; b++) {
                int64_t f = a[b];
                for (int t = 0; t < nt[b]; t++)
                    for (int64_t r = 0; r < dur[b][(size_t)t]; r++)
                        require(sr[(size_t)f++] == (int32_t)(ts[b] + t), "kk_layout_src_row row");
            }
        }
        // durations: >= 1, the rule's saturating conversion for non-finite sums
        const int T = (int)below(8);
        std::vector<float> lg((size_t)T * 50 + 1);
        for (auto& x : lg) {
            const int k = (int)below(20);
            x = k == 0 ? std::nanf("") : k == 1 ? -std::numeric_limits<float>::infinity()
                                     : k == 2 ? std::numeric_limits<float>::infinity()
                                              : (float)((double)(int64_t)(next() % 4000) / 100.0 - 20.0);
        }
        std::vector<int64_t> dd((size_t)T + 1);
        const float spd = speeds[below(7)];
        const int rd = kk_durations_from_logits(lg.data(), T, spd, dd.data());
        require((rd == KK_OK) == (std::isfinite(spd) && spd > 0.f), "kk_durations_from_logits refusal");
        if (rd == KK_OK)
            for (int t = 0; t < T; t++) require(dd[(size_t)t] >= 1, "kk_durations_from_logits clamp");
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: host_fuzz ITERS FILE...\n");
        return 2;
    }
    const int iters = std::atoi(argv[1]);
    long read = 0, refused = 0, total = 0;
    for (int f = 2; f < argc; f++) {
        const std::vector<uint8_t> seed = read_all(argv[f]);
        const std::vector<size_t> pk = pickle_spans(seed);
        for (int i = 0; i <= iters; i++) {
            std::vector<uint8_t> m = i == 0 ? seed : mutate(seed, pk);
            total++;
            // the reader as the model file and as a voice pack (each refuses what it does not read)
            for (int as_voice = 0; as_voice < 2; as_voice++) {
                try {
                    if (as_voice) {
                        const kk::HostTensor t = kk::read_voice_pack_bytes(m, "mutant");
                        require(t.shape.size() == 3 && t.data.size() == (size_t)(t.shape[0] * t.shape[1] * t.shape[2]),
                                "voice pack shape");
                    } else {
                        auto t = kk::read_model_checkpoint_bytes(m, "mutant");
                        for (auto& kv : t) {
                            size_t n = 1;
                            for (auto d : kv.second.shape) n *= (size_t)d;
                            require(n == kv.second.data.size(), "tensor element count");
                        }
                    }
                    read++;
                } catch (const std::runtime_error&) {
                    refused++;
                }
            }
        }
    }
    fuzz_host_rules(iters * 4);
    std::printf("mutants %ld read %ld refused %ld other 0; host rules %ld ok\n", total, read, refused, g_host_ok);
    return 0;
}
