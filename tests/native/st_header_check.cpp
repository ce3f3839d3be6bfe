// CPU harness for the safetensors header parser of libanima_hip
// (anima-on-android_amd/csrc/safetensors_header.h), built by the tests with
// AddressSanitizer and UndefinedBehaviorSanitizer.
//
//   st_header_check FILE...      parse each file's header as the library
//                                does; print "ok N" or "refused: reason"
//   st_header_check --fuzz SEED N
//                                N mutated headers from a seed corpus; stop
//                                at the first header whose accepted entries
//                                break an invariant (the sanitizers stop the
//                                run at the first memory or UB error)
//
// Exit status: 0 when every file was handled (accepted or refused) and every
// fuzz case kept the invariants, 1 otherwise.
#include "safetensors_header.h"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <random>
#include <string>
#include <vector>

namespace {

using anima_hip::st::Entry;

// What an accepted header must satisfy: every tensor inside the data region
// and its byte count equal to dtype size x element count.
bool invariants_hold(const std::vector<Entry> &es, size_t data_len, std::string &why)
{
    for (const Entry &e : es) {
        if (e.begin > data_len || e.bytes > data_len - e.begin) {
            why = "tensor '" + e.name + "' outside the data region";
            return false;
        }
        unsigned __int128 n = 1;
        for (int64_t d : e.shape) {
            if (d < 0) {
                why = "negative dimension in '" + e.name + "'";
                return false;
            }
            n *= static_cast<unsigned __int128>(d);
            if (n > (static_cast<unsigned __int128>(1) << 100))
                n = static_cast<unsigned __int128>(1) << 100;  // already too large
        }
        const unsigned __int128 need = n * anima_hip::st::dtype_bytes(e.dtype);
        if (need != e.bytes) {
            why = "byte count of '" + e.name + "' does not match its shape";
            return false;
        }
    }
    return true;
}

// Parse a whole file the way anima_hip_weights_open frames it.
int check_file(const char *path)
{
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        std::printf("%s: cannot open\n", path);
        return 1;
    }
    std::vector<char> buf((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    if (buf.size() < 8) {
        std::printf("%s: refused: too short\n", path);
        return 0;
    }
    uint64_t hl = 0;
    for (int i = 7; i >= 0; --i)
        hl = (hl << 8) | static_cast<unsigned char>(buf[size_t(i)]);
    if (hl > buf.size() - 8) {
        std::printf("%s: refused: header length beyond the file\n", path);
        return 0;
    }
    // The header goes into its own exact-size allocation so that any read
    // past its end is caught by AddressSanitizer.
    std::vector<char> hdr(buf.begin() + 8, buf.begin() + 8 + long(hl));
    const size_t data_len = buf.size() - 8 - size_t(hl);
    std::vector<Entry> es;
    std::string err, why;
    if (!anima_hip::st::parse_header(hdr.data(), hdr.data() + hdr.size(), data_len, es, err)) {
        std::printf("%s: refused: %s\n", path, err.c_str());
        return 0;
    }
    if (!invariants_hold(es, data_len, why)) {
        std::printf("%s: ACCEPTED A BAD HEADER: %s\n", path, why.c_str());
        return 1;
    }
    std::printf("%s: ok %zu\n", path, es.size());
    return 0;
}

const char *const kSeeds[] = {
    "{\"a\": {\"dtype\": \"F32\", \"shape\": [2, 4], \"data_offsets\": [0, 32]}}",
    "{\"__metadata__\": {\"format\": \"pt\", \"x\": [1, [2, {\"y\": null}], true, 1.5e3]},"
    " \"b\": {\"dtype\": \"BF16\", \"shape\": [16], \"data_offsets\": [0, 32]},"
    " \"c\": {\"dtype\": \"F16\", \"shape\": [], \"data_offsets\": [32, 34], \"extra\": \"s\\\"q\"}}",
    "{\"w\": {\"shape\": [4611686018427387904], \"dtype\": \"F32\", \"data_offsets\": [0, 0]}}",
    "{\"__metadata__\": [[[[[[[[[[[[[[[[]]]]]]]]]]]]]]]]}",
    "{}",
};

// One random edit of a header: flip, insert, delete or duplicate bytes, or
// splice in a token that steers the parser into its edge cases.
void mutate(std::string &s, std::mt19937_64 &rng)
{
    static const char *const tokens[] = {"[", "]", "{", "}", ",", ":", "\"", "\\", "-",
                                         "9223372036854775807", "18446744073709551616",
                                         "4611686018427387904", "\"__metadata__\"", "\"shape\"",
                                         "\"dtype\"", "\"data_offsets\"", "\"BF16\"", "0", " "};
    const size_t ntok = sizeof(tokens) / sizeof(tokens[0]);
    const int op = int(rng() % 5);
    const size_t pos = s.empty() ? 0 : size_t(rng() % (s.size() + 1));
    switch (op) {
    case 0:
        if (!s.empty())
            s[pos % s.size()] = char(rng() % 256);
        break;
    case 1:
        s.insert(pos, tokens[rng() % ntok]);
        break;
    case 2:
        if (!s.empty())
            s.erase(pos % s.size(), 1 + size_t(rng() % 4));
        break;
    case 3: {
        const size_t n = size_t(rng() % 64);
        s.insert(pos, std::string(n, rng() % 2 ? '[' : '{'));
        break;
    }
    default:
        if (!s.empty() && s.size() < 4096) {
            const size_t a = pos % s.size(), n = 1 + size_t(rng() % 16);
            s.insert(pos, s.substr(a, n));
        }
        break;
    }
}

int fuzz(uint64_t seed, long n)
{
    std::mt19937_64 rng(seed);
    const size_t nseeds = sizeof(kSeeds) / sizeof(kSeeds[0]);
    long accepted = 0;
    for (long i = 0; i < n; ++i) {
        std::string h = kSeeds[rng() % nseeds];
        const int edits = 1 + int(rng() % 6);
        for (int e = 0; e < edits; ++e)
            mutate(h, rng);
        if (rng() % 16 == 0)  // a deeply nested value in __metadata__
            h = "{\"__metadata__\": " + std::string(size_t(60 + rng() % 40), '[') + "}";
        std::vector<char> hdr(h.begin(), h.end());
        const size_t data_len = size_t(rng() % 128);
        std::vector<Entry> es;
        std::string err, why;
        if (anima_hip::st::parse_header(hdr.data(), hdr.data() + hdr.size(), data_len, es,
                                        err)) {
            ++accepted;
            if (!invariants_hold(es, data_len, why)) {
                std::printf("fuzz case %ld accepted a bad header (%s): %s\n", i, why.c_str(),
                            h.c_str());
                return 1;
            }
        }
    }
    std::printf("fuzz ok: %ld cases, %ld accepted\n", n, accepted);
    return 0;
}

}  // namespace

int main(int argc, char **argv)
{
    if (argc == 4 && std::strcmp(argv[1], "--fuzz") == 0)
        return fuzz(std::strtoull(argv[2], nullptr, 10), std::strtol(argv[3], nullptr, 10));
    int rc = 0;
    for (int i = 1; i < argc; ++i)
        rc |= check_file(argv[i]);
    return rc;
}
