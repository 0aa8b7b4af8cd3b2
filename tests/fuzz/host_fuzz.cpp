// Randomised inputs for the library's host-side parsers, built with AddressSanitizer and UBSan by
// tests/test_host_fuzz.py (g++, host code only): tokenizer.vocab texts (ud_tokenizer_parse /
// decode / piece) and safetensors files (ud_safetensors_open / info / read_f32), valid and
// corrupted (flipped bytes, truncation, absurd header lengths, random headers, out-of-range
// offsets).  The GPU-side entry points the parsers' loaders call are stubbed to fail here.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>
#include <unistd.h>
#include "ud_safetensors.h"
#include "ud_tokenizer.h"
int ud_set_error(int code, const char*) { return code; }
extern "C" {
int ud_encoder_get_config(const ud_encoder*, ud_encoder_config*) { return -1; }
int ud_encoder_set_weight(ud_encoder*, const char*, const float*, int64_t) { return -1; }
int ud_rnnt_set_weight(ud_rnnt*, const char*, const float*, int64_t) { return -1; }
int ud_mel_create(const float*, int32_t, const float*, ud_mel**) { return -1; }
int ud_streamer_tokens(const ud_streamer*, int32_t, int32_t*, int32_t, int32_t*) { return -1; }
}
static long st_open, st_read, tk_ok;
static std::mt19937_64 rng(12345);
static std::string rand_text(size_t n) {
    static const char* atoms[] = {"\t", "\n", "\r", "\r\n", "<0x", ">", "41", "E2", "zz", "<unk>", "\xE2\x96\x81", "a", "\xff", "\xc3\xa9", "\xe6\x97\xa5", "\xf0\x9f\x98\x80", "\xed\xa0\x80", "\xc0", "-1.5", " "};
    std::string s;
    while (s.size() < n) s += atoms[rng() % (sizeof atoms / sizeof *atoms)];
    return s;
}
static void fuzz_tok(int iters) {
    for (int it = 0; it < iters; it++) {
        std::string t = rand_text(rng() % 400);
        if (rng() % 4 == 0) for (auto& c : t) if (rng() % 10 == 0) c = (char)(rng() & 0xff);
        ud_tokenizer* tk = nullptr;
        if (ud_tokenizer_parse(t.data(), (int64_t)t.size(), &tk) != 0) continue;
        tk_ok++;
        int32_t n = 0; ud_tokenizer_size(tk, &n);
        for (int r = 0; r < 8; r++) {
            std::vector<int32_t> ids(rng() % 50);
            for (auto& x : ids) x = (int32_t)(rng() % (n + 6)) - 3;
            int64_t len = 0;
            ud_tokenizer_decode(tk, ids.data(), (int32_t)ids.size(), nullptr, 0, &len);
            std::vector<char> buf((size_t)len + 1);
            int64_t cap = rng() % 2 ? len : (int64_t)(rng() % (len + 1));
            ud_tokenizer_decode(tk, ids.data(), (int32_t)ids.size(), buf.data(), cap, &len);
        }
        for (int32_t i = -1; i <= n; i++) { char b[8]; int64_t l; ud_tokenizer_piece(tk, i, b, 8, &l); }
        ud_tokenizer_destroy(tk);
    }
}
static std::string st_file(const std::string& header, const std::string& data) {
    std::string f(8, '\0');
    uint64_t n = header.size();
    memcpy(&f[0], &n, 8);
    return f + header + data;
}
static void fuzz_st(int iters, const char* path) {
    const char* dts[] = {"F32", "F16", "BF16", "I64", "U8", "F64", "\"", ""};
    for (int it = 0; it < iters; it++) {
        std::string h = "{";
        int nt = rng() % 4;
        size_t off = 0;
        std::string data;
        for (int k = 0; k < nt; k++) {
            int nd = rng() % 4;
            std::string shp = "[";
            int64_t el = 1;
            for (int d = 0; d < nd; d++) { int v = rng() % 5; el *= v; shp += (d ? "," : "") + std::to_string(v); }
            shp += "]";
            const char* dt = dts[rng() % 8];
            int64_t bytes = el * 4;
            size_t b0 = off, b1 = off + (size_t)bytes + (rng() % 5 == 0 ? rng() % 7 : 0);
            if (rng() % 6 == 0) b1 = (size_t)(rng() % 1000);
            h += (k ? "," : "") + std::string("\"t") + std::to_string(k) + "\":{\"dtype\":\"" + dt + "\",\"shape\":" + shp +
                 ",\"data_offsets\":[" + std::to_string(b0) + "," + std::to_string(b1) + "]}";
            off = b1 > off ? b1 : off;
        }
        if (rng() % 3 == 0) h += std::string(nt ? "," : "") + "\"__metadata__\":{\"format\":\"pt\"}";
        h += "}";
        data.assign(off + rng() % 3, '\x3f');
        std::string f = st_file(h, data);
        int mode = rng() % 6;
        if (mode == 0) for (auto& c : f) { if (rng() % 20 == 0) c = (char)(rng() & 0xff); }
        else if (mode == 1 && f.size() > 1) f.resize(rng() % f.size());
        else if (mode == 2 && f.size() >= 8) { uint64_t big = rng(); memcpy(&f[0], &big, 8); }
        else if (mode == 3) { std::string r = rand_text(rng() % 200); f = st_file(r, data); }
        FILE* o = fopen(path, "wb"); fwrite(f.data(), 1, f.size(), o); fclose(o);
        ud_safetensors* st = nullptr;
        if (ud_safetensors_open(path, &st) != 0) continue;
        st_open++;
        int32_t c = ud_safetensors_count(st);
        for (int32_t i = -1; i <= c; i++) {
            const char* nm = ud_safetensors_name(st, i);
            if (!nm) continue;
            int32_t dt, ndim; int64_t shape[8];
            if (ud_safetensors_info(st, nm, &dt, shape, &ndim) != 0) continue;
            int64_t cnt = 1; for (int d = 0; d < ndim; d++) cnt *= shape[d];
            std::vector<float> buf((size_t)(cnt > 0 ? cnt : 1));
            if (ud_safetensors_read_f32(st, nm, buf.data(), cnt) == 0) st_read++;
            ud_safetensors_read_f32(st, nm, buf.data(), cnt > 0 ? cnt - 1 : 0);
        }
        ud_safetensors_info(st, "nope", nullptr, nullptr, nullptr);
        ud_safetensors_close(st);
    }
}
int main(int argc, char** argv) {
    int iters = argc > 1 ? atoi(argv[1]) : 20000;
    fuzz_tok(iters);
    char path[] = "/tmp/fuzzstXXXXXX";
    int fd = mkstemp(path); close(fd);
    fuzz_st(iters, path);
    unlink(path);
    printf("fuzz ok: %d iterations each; tokenizers parsed %ld, safetensors opened %ld, tensors read %ld\n", iters, tk_ok, st_open, st_read);
    return 0;
}
