// SentencePiece detokenizer (include/ud_tokenizer.h): host code, no device work.
//
// SentencePieceDecoder (Sources/DictatorCore/Decoding/SentencePiece.swift:5-31): vocabulary
// parsing (:8-13) and decode (:17-30), with the UTF-8 repair of Swift's String(decoding:as:).
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/ud_tokenizer.h"

int ud_set_error(int code, const char* msg);   // encoder.hip

struct ud_tokenizer {
    std::vector<std::string> pieces;
};

namespace {

int fail(int code, const char* msg) { return ud_set_error(code, msg); }

// A line's piece: its first non-empty tab-separated field (SentencePiece.swift:12, Swift's split
// omits empty fields), "" when the line is all tabs.
std::string first_field(const char* p, size_t n) {
    size_t i = 0;
    while (i < n && p[i] == '\t') i++;
    size_t j = i;
    while (j < n && p[j] != '\t') j++;
    return std::string(p + i, j - i);
}

// "<0xHH>" with two hex digits -> the byte (SentencePiece.swift:21)
bool byte_piece(const std::string& p, unsigned char& b) {
    if (p.size() != 6 || p.compare(0, 3, "<0x") != 0 || p[5] != '>') return false;
    int v = 0;
    for (int k = 3; k < 5; k++) {
        const char c = p[k];
        int d;
        if (c >= '0' && c <= '9') d = c - '0';
        else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
        else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
        else return false;
        v = v * 16 + d;
    }
    b = (unsigned char)v;
    return true;
}

// Bytes of a well-formed UTF-8 sequence starting at s[i] (Unicode Table 3-7), or, for an
// ill-formed one, the length of its maximal subpart (at least 1) with ok = false.
size_t utf8_step(const unsigned char* s, size_t n, size_t i, bool& ok) {
    const unsigned char c = s[i];
    ok = true;
    if (c < 0x80) return 1;
    int need;
    unsigned char lo = 0x80, hi = 0xBF;   // bounds of the second byte
    if (c >= 0xC2 && c <= 0xDF) need = 1;
    else if (c == 0xE0) { need = 2; lo = 0xA0; }
    else if (c >= 0xE1 && c <= 0xEC) need = 2;
    else if (c == 0xED) { need = 2; hi = 0x9F; }
    else if (c >= 0xEE && c <= 0xEF) need = 2;
    else if (c == 0xF0) { need = 3; lo = 0x90; }
    else if (c >= 0xF1 && c <= 0xF3) need = 3;
    else if (c == 0xF4) { need = 3; hi = 0x8F; }
    else { ok = false; return 1; }            // 80..BF, C0, C1, F5..FF: never a lead byte
    size_t k = 1;
    for (; k <= (size_t)need; k++) {
        if (i + k >= n) { ok = false; return k; }
        const unsigned char d = s[i + k];
        const unsigned char l = k == 1 ? lo : 0x80, h = k == 1 ? hi : 0xBF;
        if (d < l || d > h) { ok = false; return k; }
    }
    return k;
}

std::string decode_ids(const ud_tokenizer* t, const int32_t* ids, int32_t n) {
    static const char kMark[] = "\xE2\x96\x81";   // U+2581
    std::string bytes;
    for (int32_t i = 0; i < n; i++) {
        const int32_t id = ids[i];
        if (id < 0 || id >= (int32_t)t->pieces.size()) continue;
        const std::string& p = t->pieces[id];
        unsigned char b;
        if (byte_piece(p, b)) {
            bytes.push_back((char)b);
        } else if (p == "<unk>" || p == "<s>" || p == "</s>" || p == "<pad>") {
            continue;
        } else {
            for (size_t k = 0; k < p.size();) {
                if (p.compare(k, 3, kMark) == 0) { bytes.push_back(' '); k += 3; }
                else bytes.push_back(p[k++]);
            }
        }
    }
    // UTF-8 repair: each maximal ill-formed subpart becomes U+FFFD
    std::string text;
    text.reserve(bytes.size());
    const unsigned char* s = reinterpret_cast<const unsigned char*>(bytes.data());
    for (size_t i = 0; i < bytes.size();) {
        bool ok;
        const size_t k = utf8_step(s, bytes.size(), i, ok);
        if (ok) text.append(bytes, i, k);
        else text.append("\xEF\xBF\xBD");
        i += k;
    }
    if (!text.empty() && text[0] == ' ') text.erase(0, 1);
    return text;
}

int copy_out(const std::string& v, char* out, int64_t cap, int64_t* len) {
    if (cap < 0 || (cap > 0 && !out)) return fail(UD_ERR_INVALID, "ud_tokenizer: bad output buffer");
    const int64_t m = (int64_t)v.size() < cap ? (int64_t)v.size() : cap;
    if (m > 0) memcpy(out, v.data(), (size_t)m);
    if (len) *len = (int64_t)v.size();
    return UD_OK;
}

}  // namespace

extern "C" UD_API int ud_tokenizer_parse(const char* text, int64_t bytes, ud_tokenizer** out) {
    if (!out || bytes < 0 || (bytes > 0 && !text)) return fail(UD_ERR_INVALID, "ud_tokenizer_parse: bad argument");
    *out = nullptr;
    // the file must be UTF-8 (String(contentsOf:encoding: .utf8) throws otherwise)
    const unsigned char* u = reinterpret_cast<const unsigned char*>(text);
    for (size_t i = 0; i < (size_t)bytes;) {
        bool ok;
        i += utf8_step(u, (size_t)bytes, i, ok);
        if (!ok) return fail(UD_ERR_INVALID, "ud_tokenizer_parse: the vocabulary is not UTF-8");
    }
    ud_tokenizer* t = new (std::nothrow) ud_tokenizer;
    if (!t) return fail(UD_ERR_NOMEM, "ud_tokenizer_parse: allocation failed");
    // lines end at a '\n' not preceded by '\r'; empty lines are dropped (SentencePiece.swift:10-11)
    size_t start = 0;
    const size_t n = (size_t)bytes;
    for (size_t i = 0; i <= n; i++) {
        const bool end = i == n || (text[i] == '\n' && !(i > 0 && text[i - 1] == '\r'));
        if (!end) continue;
        if (i > start) t->pieces.push_back(first_field(text + start, i - start));
        start = i + 1;
    }
    *out = t;
    return UD_OK;
}

extern "C" UD_API int ud_tokenizer_load(const char* vocab_path, ud_tokenizer** out) {
    if (!vocab_path || !out) return fail(UD_ERR_INVALID, "ud_tokenizer_load: null argument");
    *out = nullptr;
    FILE* f = fopen(vocab_path, "rb");
    if (!f) {
        char buf[512];
        snprintf(buf, sizeof buf, "ud_tokenizer_load: cannot open %s", vocab_path);
        return fail(UD_ERR_INVALID, buf);
    }
    std::string text;
    char chunk[1 << 16];
    size_t got;
    while ((got = fread(chunk, 1, sizeof chunk, f)) > 0) text.append(chunk, got);
    const bool err = ferror(f) != 0;
    fclose(f);
    if (err) return fail(UD_ERR_INVALID, "ud_tokenizer_load: read error");
    return ud_tokenizer_parse(text.data(), (int64_t)text.size(), out);
}

extern "C" UD_API void ud_tokenizer_destroy(ud_tokenizer* t) { delete t; }

extern "C" UD_API int ud_tokenizer_size(const ud_tokenizer* t, int32_t* size) {
    if (!t || !size) return fail(UD_ERR_INVALID, "ud_tokenizer_size: null argument");
    *size = (int32_t)t->pieces.size();
    return UD_OK;
}

extern "C" UD_API int ud_tokenizer_piece(const ud_tokenizer* t, int32_t id, char* out, int64_t cap, int64_t* len) {
    if (!t) return fail(UD_ERR_INVALID, "ud_tokenizer_piece: null tokenizer");
    if (id < 0 || id >= (int32_t)t->pieces.size()) return fail(UD_ERR_SHAPE, "ud_tokenizer_piece: id out of range");
    return copy_out(t->pieces[id], out, cap, len);
}

extern "C" UD_API int ud_tokenizer_decode(const ud_tokenizer* t, const int32_t* ids, int32_t n, char* out, int64_t cap,
                                          int64_t* len) {
    if (!t || n < 0 || (n > 0 && !ids)) return fail(UD_ERR_INVALID, "ud_tokenizer_decode: bad argument");
    return copy_out(decode_ids(t, ids, n), out, cap, len);
}

extern "C" UD_API int ud_streamer_text(const ud_streamer* s, int32_t id, const ud_tokenizer* t, char* out, int64_t cap,
                                       int64_t* len) {
    if (!s || !t) return fail(UD_ERR_INVALID, "ud_streamer_text: null argument");
    int32_t count = 0;
    int rc = ud_streamer_tokens(s, id, nullptr, 0, &count);
    if (rc != UD_OK) return rc;
    std::vector<int32_t> ids((size_t)count);
    if (count > 0 && (rc = ud_streamer_tokens(s, id, ids.data(), count, &count)) != UD_OK) return rc;
    return ud_tokenizer_decode(t, ids.data(), (int32_t)ids.size(), out, cap, len);
}
