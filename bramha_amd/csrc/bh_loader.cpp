// bh_loader.cpp — the reference's on-disk model directory → device upload.
//
// Format (written by src/bin/quantize_model.rs:284-306, read by the manifest branch of
// src/storage/tensor_db.rs:623-724): `manifest.json` holds `layers`, a map of layer metadata
// {layer_id, shape, compression_format, checksum, ...}; each tensor lives in a shard file named
// after the layer id with '.' replaced by '_':
//   Int4PerChannel  `{id}_u4.bin`  u8 [n][k/2] (quantize_to_int4 bytes) and, as the separate
//                   layer `{id}.scale`, `{id}_scale.bin` f32 [n];
//   Int8Linear      `{id}_i8.bin`  i8 [n][k] and `{id}_scale.bin` f32 [n];
//   None            `{id}.bin`     f32, row-major.
// The candidate file names and their order are the reference's (tensor_db.rs:631-651); a
// non-empty checksum is the SHA-256 of the shard file, and a mismatch is an error (the reference
// panics, :662-676). The reference maps Int8Linear shards to an F32 tensor (:682-691), which reads
// int8 bytes as floats; here they load as BH_Q8_ROW. Svd, dictionary, differential and GGUF
// layers are not part of this path and are reported as unsupported.
//
// Shards are memory-mapped and handed to bh_model_set_weight, which repacks and uploads them.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "bramha_hip.h"

namespace {

// ------------------------------------------------------------ a JSON subset reader
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    bool b = false;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;
    const Json* get(const char* k) const {
        if (kind != OBJ) return nullptr;
        auto it = obj.find(k);
        return it == obj.end() ? nullptr : &it->second;
    }
};

struct Parser {
    const char* p;
    const char* e;
    std::string err;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    bool str(std::string& out) {
        if (p >= e || *p != '"') return fail("expected a string");
        ++p;
        while (p < e && *p != '"') {
            if (*p == '\\') {
                if (++p >= e) return fail("bad escape");
                switch (*p) {
                    case 'n': out += '\n'; break;
                    case 't': out += '\t'; break;
                    case 'r': out += '\r'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u': {  // keep ASCII code points; others become '?'
                        if (e - p < 5) return fail("bad \\u escape");
                        const unsigned v = (unsigned)std::strtoul(std::string(p + 1, p + 5).c_str(), nullptr, 16);
                        out += v < 0x80 ? (char)v : '?';
                        p += 4;
                        break;
                    }
                    default: out += *p;
                }
                ++p;
            } else {
                out += *p++;
            }
        }
        if (p >= e) return fail("unterminated string");
        ++p;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= e) return fail("unexpected end");
        if (*p == '{') {
            v.kind = Json::OBJ;
            ++p;
            ws();
            if (p < e && *p == '}') return ++p, true;
            for (;;) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (p >= e || *p != ':') return fail("expected ':'");
                ++p;
                if (!value(v.obj[k], depth + 1)) return false;
                ws();
                if (p < e && *p == ',') { ++p; continue; }
                if (p < e && *p == '}') return ++p, true;
                return fail("expected ',' or '}'");
            }
        }
        if (*p == '[') {
            v.kind = Json::ARR;
            ++p;
            ws();
            if (p < e && *p == ']') return ++p, true;
            for (;;) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                ws();
                if (p < e && *p == ',') { ++p; continue; }
                if (p < e && *p == ']') return ++p, true;
                return fail("expected ',' or ']'");
            }
        }
        if (*p == '"') {
            v.kind = Json::STR;
            return str(v.str);
        }
        if (e - p >= 4 && !std::strncmp(p, "null", 4)) return p += 4, true;
        if (e - p >= 4 && !std::strncmp(p, "true", 4)) return v.kind = Json::BOOL, v.b = true, p += 4, true;
        if (e - p >= 5 && !std::strncmp(p, "false", 5)) return v.kind = Json::BOOL, v.b = false, p += 5, true;
        char* end = nullptr;
        const std::string tok(p, std::min<size_t>(64, (size_t)(e - p)));
        v.num = std::strtod(tok.c_str(), &end);
        if (end == tok.c_str()) return fail("bad value");
        v.kind = Json::NUM;
        p += end - tok.c_str();
        return true;
    }
};

// ------------------------------------------------------------ SHA-256 (FIPS 180-4)
struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void block(const uint8_t* m) {
        static const uint32_t K[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)m[4 * i] << 24 | (uint32_t)m[4 * i + 1] << 16 | (uint32_t)m[4 * i + 2] << 8 | m[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    std::string hex(const uint8_t* data, size_t n) {
        size_t i = 0;
        for (; i + 64 <= n; i += 64) block(data + i);
        uint8_t tail[128] = {0};
        const size_t r = n - i;
        std::memcpy(tail, data + i, r);
        tail[r] = 0x80;
        const size_t tl = r < 56 ? 64 : 128;
        const uint64_t bits = (uint64_t)n * 8;
        for (int k = 0; k < 8; ++k) tail[tl - 1 - k] = (uint8_t)(bits >> (8 * k));
        block(tail);
        if (tl == 128) block(tail + 64);
        char out[65];
        for (int k = 0; k < 8; ++k) std::snprintf(out + 8 * k, 9, "%08x", h[k]);
        return std::string(out, 64);
    }
};

// ------------------------------------------------------------ read-only mapped shard
struct Mapped {
    void* p = nullptr;
    size_t n = 0;
    ~Mapped() {
        if (p && n) munmap(p, n);
    }
    bool open(const std::string& path) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) return false;
        struct stat st;
        if (fstat(fd, &st) != 0) {
            ::close(fd);
            return false;
        }
        n = (size_t)st.st_size;
        if (n) p = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (p == MAP_FAILED) p = nullptr, n = 0;
        return n == 0 || p;
    }
};

bool exists(const std::string& path) {
    struct stat st;
    return stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

std::string safe_name(const std::string& id) {
    std::string s = id;
    for (char& c : s)
        if (c == '.') c = '_';
    return s;
}

std::string format_name(const Json* f) {
    if (!f) return "None";
    if (f->kind == Json::STR) return f->str;
    if (f->kind == Json::OBJ && !f->obj.empty()) return f->obj.begin()->first;  // e.g. {"Differential": {...}}
    return "None";
}

}  // namespace

// Both have C linkage: they are declared next to the C ABI in bh_model.cpp.
extern "C" const char* model_last_error(bh_model* m);  // bh_model.cpp
extern "C" int model_load_dir(bh_model* m, const char* dir, int* n_loaded, std::string* err);

// Load every tensor of a model directory in the reference's format into `m` (see the file
// header). Returns BH_OK with *n_loaded tensors set; tensors the model does not use are skipped.
int model_load_dir(bh_model* m, const char* dir, int* n_loaded, std::string* err) {
    *n_loaded = 0;
    const std::string root(dir);
    Mapped mf;
    if (!mf.open(root + "/manifest.json") || !mf.p) {
        *err = "cannot read " + root + "/manifest.json";
        return BH_ERR_NOT_FOUND;
    }
    Json man;
    Parser ps{(const char*)mf.p, (const char*)mf.p + mf.n, {}};
    if (!ps.value(man, 0)) {
        *err = "manifest.json: " + ps.err;
        return BH_ERR_INVALID;
    }
    const Json* layers = man.get("layers");
    if (!layers || layers->kind != Json::OBJ) {
        *err = "manifest.json has no layers map";
        return BH_ERR_INVALID;
    }
    for (const auto& kv : layers->obj) {
        const Json& meta = kv.second;
        const Json* idj = meta.get("layer_id");
        const std::string id = idj && idj->kind == Json::STR ? idj->str : kv.first;
        if (id.size() > 6 && id.compare(id.size() - 6, 6, ".scale") == 0) continue;  // read with its weight
        const std::string fmt = format_name(meta.get("compression_format"));
        const std::string sn = safe_name(id);
        std::vector<std::string> cand;
        if (fmt == "Int4PerChannel") cand = {sn + "_u4.bin", sn + "_scale.bin", sn + ".bin"};
        else if (fmt == "Int8Linear") cand = {sn + "_i8.bin", sn + "_scale.bin", sn + ".bin"};
        else if (fmt == "None") cand = {sn + ".bin"};
        else {
            *err = "layer " + id + ": compression format " + fmt + " is not supported by this backend";
            return BH_ERR_UNSUPPORTED;
        }
        std::string path;
        for (const auto& c : cand)
            if (exists(root + "/" + c)) {
                path = root + "/" + c;
                break;
            }
        if (path.empty()) continue;  // the reference warns and skips a missing shard
        Mapped data;
        if (!data.open(path)) {
            *err = "cannot map " + path;
            return BH_ERR_INVALID;
        }
        const Json* ck = meta.get("checksum");
        if (ck && ck->kind == Json::STR && !ck->str.empty()) {
            const std::string got = Sha256().hex((const uint8_t*)data.p, data.n);
            if (got != ck->str) {
                *err = "checksum mismatch for tensor shard " + path + ": expected " + ck->str + ", actual " + got;
                return BH_ERR_INVALID;
            }
        }
        const bool quant = fmt == "Int4PerChannel" || fmt == "Int8Linear";
        const bool is_q = quant && path.size() > 7 &&
                          (path.compare(path.size() - 7, 7, "_u4.bin") == 0 || path.compare(path.size() - 7, 7, "_i8.bin") == 0);
        Mapped scales;
        if (is_q && !scales.open(root + "/" + sn + "_scale.bin")) {
            *err = "layer " + id + ": missing " + sn + "_scale.bin";
            return BH_ERR_NOT_FOUND;
        }
        const int rc = bh_model_set_weight(m, id.c_str(), data.p, data.n, is_q ? scales.p : nullptr, is_q ? scales.n : 0);
        if (rc == BH_ERR_NOT_FOUND) continue;  // a tensor this decoder does not use
        if (rc != BH_OK) {
            *err = "layer " + id + ": " + std::string(model_last_error(m));
            return rc;
        }
        ++*n_loaded;
    }
    return BH_OK;
}
