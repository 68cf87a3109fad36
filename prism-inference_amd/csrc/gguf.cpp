// gguf.cpp -- GGUF v3 tensor index for packed weights, and the lossless PQ2 -> PTQ1 export.
//
// The reader validates the header, the metadata table and the tensor descriptors of a
// GGUF file under a bounded policy, and resolves every tensor's absolute extent (the
// behaviour of tools/gguf/src/stream.rs:349-611: read_header, read_metadata_table,
// read_tensor_table, resolve_tensor_offsets).  Tensor payloads are read only on request,
// straight into a weight upload.  The export rewrites every PQ2 (142) tensor of a Prism
// dialect file as PTQ1 (143) with an exact re-expansion check and copies every other
// tensor verbatim (tools/gguf/src/export.rs:130-318).  Host code only: nothing here
// touches the GPU except prism_hip_weight_from_gguf, which hands the bytes to
// prism_hip_weight_acquire.
#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <vector>

#include <sys/stat.h>

#include "prism_hip.h"

namespace {

// ---- type table (tools/gguf/src/inspect.rs:68-117) -----------------------------------
bool type_layout(uint32_t id, bool prism, uint64_t *block, uint64_t *bytes) {
    struct Row {
        uint32_t id;
        uint64_t block, bytes;
    };
    static const Row rows[] = {
        {0, 1, 4},     {1, 1, 2},     {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
        {8, 32, 34},   {9, 32, 36},   {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {16, 256, 66}, {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
        {20, 32, 18},  {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
        {26, 1, 4},    {27, 1, 8},    {28, 1, 8},     {29, 256, 56},  {30, 1, 2},     {34, 256, 54},
        {35, 256, 66}, {39, 32, 17},  {40, 64, 36},   {41, 128, 18},  {42, 64, 18},
    };
    for (const Row &r : rows)
        if (r.id == id) {
            *block = r.block;
            *bytes = r.bytes;
            return true;
        }
    if (prism && (id == 142 || id == 143)) {
        *block = 128;
        *bytes = id == 142 ? 34 : 28;
        return true;
    }
    return false;
}

// Scalar metadata widths (inspect.rs:127-135); 8 = string, 9 = array.
int scalar_width(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
    }
}

bool utf8_valid(const unsigned char *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const unsigned char c = s[i];
        size_t len;
        uint32_t cp;
        if (c < 0x80) {
            ++i;
            continue;
        } else if ((c & 0xe0) == 0xc0) {
            len = 2;
            cp = c & 0x1f;
        } else if ((c & 0xf0) == 0xe0) {
            len = 3;
            cp = c & 0x0f;
        } else if ((c & 0xf8) == 0xf0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (size_t k = 1; k < len; ++k) {
            if ((s[i + k] & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && (cp < 0x10000 || cp > 0x10ffff)) ||
            (cp >= 0xd800 && cp <= 0xdfff))
            return false;
        i += len;
    }
    return true;
}

struct Meta {
    uint32_t type = 0;       // GGUF value type (8 string, 9 array)
    uint32_t elem = 0;       // array element type
    uint64_t count = 0;      // array element count
    uint64_t value_pos = 0;  // file offset of the scalar value (after its type tag)
    uint64_t u = 0;          // unsigned / bool scalars
    int64_t i = 0;           // signed scalars
    double f = 0.0;          // float scalars
    std::string s;           // string scalar
    std::vector<std::string> strings;  // retained string array
    bool retained = true;
};

struct Tensor {
    uint32_t type = 0, ndims = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint64_t relative_offset = 0, offset = 0, bytes = 0, elements = 0;
    uint64_t type_pos = 0;  // file offset of the descriptor's type id
};

class Reader {
  public:
    Reader(FILE *f, uint64_t file_bytes, const prism_gguf_policy &p) : f_(f), file_bytes_(file_bytes), p_(p) {
        budget_ = p.metadata_budget;
    }
    uint64_t pos() const { return pos_; }
    uint64_t budget() const { return budget_; }
    bool charge(uint64_t n) {
        if (n > budget_) return false;
        budget_ -= n;
        return true;
    }
    bool need(uint64_t n) const { return n <= file_bytes_ - pos_; }
    bool bytes(void *dst, uint64_t n) {
        if (!need(n)) return false;
        if (n && std::fread(dst, 1, n, f_) != n) return false;
        pos_ += n;
        return true;
    }
    template <typename T>
    bool get(T *v) {
        return bytes(v, sizeof(T));  // little-endian host
    }
    bool skip(uint64_t n) {
        if (!need(n)) return false;
        if (std::fseek(f_, static_cast<long>(pos_ + n), SEEK_SET) != 0) return false;
        pos_ += n;
        return true;
    }
    // A length-prefixed string: bounded, charged, no interior NUL when asked, UTF-8.
    bool text(uint64_t limit, bool reject_nul, std::string *out) {
        uint64_t n;
        if (!get(&n) || n > limit || !need(n) || !charge(n + p_.string_overhead_bytes)) return false;
        out->resize(n);
        if (!bytes(out->data(), n)) return false;
        if (reject_nul && std::memchr(out->data(), 0, n)) return false;
        return utf8_valid(reinterpret_cast<const unsigned char *>(out->data()), n);
    }

  private:
    FILE *f_;
    uint64_t file_bytes_, pos_ = 0, budget_;
    const prism_gguf_policy &p_;
};

}  // namespace

struct prism_gguf {
    std::string path;
    uint32_t version = 0;
    uint64_t alignment = 0, data_offset = 0, remaining_budget = 0, file_bytes = 0;
    std::map<std::string, Meta> metadata;
    std::map<std::string, Tensor> tensors;
    std::vector<const std::string *> tensor_names, metadata_keys;  // name order
    std::string error;
};

namespace {

thread_local std::string g_last_error;

int bad(prism_gguf *g, const char *what) {
    if (g) g->error = what;
    g_last_error = what;
    return PRISM_ERR_INVALID_INPUT;
}

bool read_scalar(Reader &r, uint32_t t, const prism_gguf_policy &p, Meta *m) {
    switch (t) {
    case 0: { uint8_t v; if (!r.get(&v)) return false; m->u = v; return true; }
    case 1: { int8_t v; if (!r.get(&v)) return false; m->i = v; return true; }
    case 2: { uint16_t v; if (!r.get(&v)) return false; m->u = v; return true; }
    case 3: { int16_t v; if (!r.get(&v)) return false; m->i = v; return true; }
    case 4: { uint32_t v; if (!r.get(&v)) return false; m->u = v; return true; }
    case 5: { int32_t v; if (!r.get(&v)) return false; m->i = v; return true; }
    case 6: {
        float v;
        if (!r.get(&v) || (p.reject_nonfinite_floats && !std::isfinite(v))) return false;
        m->f = v;
        return true;
    }
    case 7: { uint8_t v; if (!r.get(&v) || v > 1) return false; m->u = v; return true; }
    case 10: { uint64_t v; if (!r.get(&v)) return false; m->u = v; return true; }
    case 11: { int64_t v; if (!r.get(&v)) return false; m->i = v; return true; }
    case 12: {
        double v;
        if (!r.get(&v) || (p.reject_nonfinite_floats && !std::isfinite(v))) return false;
        m->f = v;
        return true;
    }
    default: return false;
    }
}

// read_array (stream.rs:390-484): string arrays retained up to the policy's byte cap,
// scalar arrays validated and skipped (booleans byte by byte); nested arrays rejected.
bool read_array(Reader &r, const prism_gguf_policy &p, Meta *m, uint64_t *retained_strings) {
    if (!r.get(&m->elem) || !r.get(&m->count) || m->count > p.max_array_items) return false;
    if (m->elem == 8) {
        if (m->count > UINT64_MAX / 8 || !r.need(m->count * 8)) return false;
        m->retained = p.retain_string_arrays != 0;
        std::string s;
        for (uint64_t k = 0; k < m->count; ++k) {
            if (!r.text(p.max_array_string_bytes, p.reject_interior_nul_strings != 0, &s)) return false;
            if (m->retained) {
                *retained_strings += s.size();
                if (p.max_retained_string_array_bytes && *retained_strings > p.max_retained_string_array_bytes)
                    return false;
                m->strings.push_back(s);
            }
        }
        return true;
    }
    const int w = scalar_width(m->elem);
    if (!w || m->count > UINT64_MAX / w) return false;
    const uint64_t payload = m->count * w;
    if (!r.need(payload)) return false;
    m->retained = false;
    if (p.charge_skipped_scalar_arrays && !r.charge(payload)) return false;
    if (m->elem == 7) {
        uint8_t buf[1024];
        for (uint64_t left = payload; left;) {
            const uint64_t step = left < sizeof(buf) ? left : sizeof(buf);
            if (!r.bytes(buf, step)) return false;
            for (uint64_t k = 0; k < step; ++k)
                if (buf[k] > 1) return false;
            left -= step;
        }
        return true;
    }
    return r.skip(payload);
}

int parse(prism_gguf *g, FILE *f, const prism_gguf_policy &p) {
    if (g->file_bytes < 24 || g->file_bytes > p.max_file_bytes) return bad(g, "GGUF: file size out of bounds");
    Reader r(f, g->file_bytes, p);
    // read_header (stream.rs:501-521)
    char magic[4];
    uint64_t ntensors, nmeta;
    if (!r.bytes(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return bad(g, "GGUF: bad magic");
    if (!r.get(&g->version) || !(g->version == 3 || (p.allow_v2 && g->version == 2)))
        return bad(g, "GGUF: unsupported version");
    if (!r.get(&ntensors) || !r.get(&nmeta)) return bad(g, "GGUF: truncated header");
    if ((!p.allow_zero_tensors && ntensors == 0) || (!p.allow_zero_metadata && nmeta == 0) ||
        ntensors > p.max_tensors || nmeta > p.max_metadata)
        return bad(g, "GGUF: tensor or metadata count out of bounds");
    // read_metadata_table (stream.rs:523-565)
    uint64_t retained_strings = 0;
    for (uint64_t k = 0; k < nmeta; ++k) {
        std::string key;
        if (!r.charge(p.kv_overhead_bytes) || !r.text(p.max_key_bytes, p.reject_interior_nul_keys != 0, &key) ||
            key.empty() || g->metadata.count(key))
            return bad(g, "GGUF: invalid or duplicate metadata key");
        Meta m;
        if (!r.get(&m.type)) return bad(g, "GGUF: truncated metadata");
        m.value_pos = r.pos();
        bool ok;
        if (m.type == 8)
            ok = r.text(p.max_string_bytes, p.reject_interior_nul_strings != 0, &m.s);
        else if (m.type == 9)
            ok = read_array(r, p, &m, &retained_strings);
        else
            ok = read_scalar(r, m.type, p, &m);
        if (!ok) return bad(g, "GGUF: invalid metadata value");
        g->metadata.emplace(std::move(key), std::move(m));
    }
    g->alignment = 32;
    auto it = g->metadata.find("general.alignment");
    if (it != g->metadata.end()) {
        const Meta &m = it->second;
        const uint64_t v = m.type == 4 ? m.u : (m.type == 5 && p.allow_positive_i32_alignment && m.i > 0) ? m.i : 0;
        if (v == 0 || (v & (v - 1)) != 0 || v > p.max_alignment) return bad(g, "GGUF: invalid general.alignment");
        g->alignment = v;
    }
    // read_tensor_table (stream.rs:567-620)
    for (uint64_t k = 0; k < ntensors; ++k) {
        std::string name;
        Tensor t;
        if (!r.charge(p.tensor_overhead_bytes) || !r.text(p.max_key_bytes, p.reject_interior_nul_keys != 0, &name) ||
            !r.get(&t.ndims) || name.empty() || g->tensors.count(name) || t.ndims < 1 || t.ndims > 4)
            return bad(g, "GGUF: invalid or duplicate tensor descriptor");
        t.elements = 1;
        for (uint32_t d = 0; d < t.ndims; ++d) {
            if (!r.get(&t.dims[d]) || t.dims[d] == 0 || t.dims[d] > static_cast<uint64_t>(INT64_MAX) ||
                t.elements > UINT64_MAX / t.dims[d])
                return bad(g, "GGUF: invalid tensor dimension");
            t.elements *= t.dims[d];
        }
        t.type_pos = r.pos();
        if (!r.get(&t.type) || !r.get(&t.relative_offset)) return bad(g, "GGUF: truncated tensor descriptor");
        if (p.allowed_types && p.allowed_type_count) {
            bool found = false;
            for (size_t a = 0; a < p.allowed_type_count; ++a) found |= p.allowed_types[a] == t.type;
            if (!found) return bad(g, "GGUF: tensor type not allowed");
        }
        uint64_t block, bb;
        if (!type_layout(t.type, p.prism_dialect != 0, &block, &bb)) return bad(g, "GGUF: unknown tensor type");
        if (t.dims[0] % block || t.relative_offset % g->alignment) return bad(g, "GGUF: misaligned tensor");
        if (t.elements / block > UINT64_MAX / bb) return bad(g, "GGUF: tensor size overflow");
        t.bytes = t.elements / block * bb;
        g->tensors.emplace(std::move(name), t);
    }
    // resolve_tensor_offsets (stream.rs:622-657)
    if (g->tensors.empty()) {
        g->data_offset = r.pos();
    } else {
        const uint64_t a = g->alignment;
        if (r.pos() > UINT64_MAX - (a - 1)) return bad(g, "GGUF: data offset overflow");
        const uint64_t aligned = (r.pos() + a - 1) / a * a;
        if (aligned > g->file_bytes) return bad(g, "GGUF: data offset past the end");
        std::vector<std::pair<uint64_t, uint64_t>> ranges;
        for (auto &kv : g->tensors) {
            Tensor &t = kv.second;
            if (t.relative_offset > UINT64_MAX - aligned) return bad(g, "GGUF: tensor offset overflow");
            t.offset = aligned + t.relative_offset;
            if (t.bytes > UINT64_MAX - t.offset || t.offset + t.bytes > g->file_bytes)
                return bad(g, "GGUF: tensor extent past the end");
            ranges.emplace_back(t.offset, t.offset + t.bytes);
        }
        std::sort(ranges.begin(), ranges.end());
        for (size_t k = 1; k < ranges.size(); ++k)
            if (ranges[k - 1].second > ranges[k].first) return bad(g, "GGUF: overlapping tensor extents");
        g->data_offset = aligned;
    }
    g->remaining_budget = r.budget();
    for (auto &kv : g->tensors) g->tensor_names.push_back(&kv.first);
    for (auto &kv : g->metadata) g->metadata_keys.push_back(&kv.first);
    return PRISM_OK;
}

const Tensor *tensor_of(const prism_gguf *g, const char *name) {
    if (!g || !name) return nullptr;
    auto it = g->tensors.find(name);
    return it == g->tensors.end() ? nullptr : &it->second;
}

void fill_info(const Tensor &t, prism_gguf_tensor *info) {
    info->type_id = t.type;
    info->ndims = t.ndims;
    for (int d = 0; d < 4; ++d) info->dims[d] = t.dims[d];
    info->relative_offset = t.relative_offset;
    info->offset = t.offset;
    info->bytes = t.bytes;
    info->elements = t.elements;
}

bool read_at(FILE *f, uint64_t off, void *dst, uint64_t n) {
    if (std::fseek(f, static_cast<long>(off), SEEK_SET) != 0) return false;
    return std::fread(dst, 1, n, f) == n;
}

// ---- PTQ1 codec (tools/ternary/src/lib.rs:135-290) -------------------------------------
bool scale_ok(const uint8_t *s) {
    const uint16_t bits = static_cast<uint16_t>(s[0] | (s[1] << 8));
    return !(bits == 0 || bits == 0x8000 || (bits & 0x7c00) == 0x7c00);
}
uint8_t pq2_code(const uint8_t *blk, int i) { return (blk[2 + i / 4] >> (2 * (i % 4))) & 3; }

// pack_ptq: a ternary PQ2 group (codes 0..2, usable scale) -> native PTQ1 bytes.
bool pack_ptq(const uint8_t *src, uint8_t *dst) {
    if (!scale_ok(src)) return false;
    for (int b = 2; b < 34; ++b)
        if (src[b] & (src[b] >> 1) & 0x55) return false;  // code 3 has no trit
    int position = 0;
    for (int width : {16, 8}) {
        const int start = position / 5;
        for (int m = 0; m < width; ++m) {
            uint32_t q = 0;
            for (int n = 0; n < 5; ++n) q = q * 3 + pq2_code(src, position + m + n * width);
            dst[start + m] = static_cast<uint8_t>((q * 256 + 242) / 243);
        }
        position += width * 5;
    }
    for (int h = 0; h < 2; ++h) {
        uint32_t q = 0;
        for (int n = 0; n < 4; ++n) q = q * 3 + pq2_code(src, 120 + h + n * 2);
        dst[24 + h] = static_cast<uint8_t>((q * 3 * 256 + 242) / 243);
    }
    dst[26] = src[0];
    dst[27] = src[1];
    return true;
}

// unpack_ptq: native PTQ1 -> PQ2, rejecting encodings that do not repack to themselves.
bool unpack_ptq(const uint8_t *src, uint8_t *dst) {
    if (!scale_ok(src + 26)) return false;
    std::memset(dst, 0, 34);
    dst[0] = src[26];
    dst[1] = src[27];
    auto digits = [](uint8_t byte, uint8_t d[5], uint32_t *value) {
        uint32_t frac = byte, v = 0;
        for (int k = 0; k < 5; ++k) {
            frac *= 3;
            d[k] = static_cast<uint8_t>(frac >> 8);
            v = v * 3 + d[k];
            frac &= 255;
        }
        *value = v;
    };
    int position = 0;
    for (int width : {16, 8}) {
        const int start = position / 5;
        for (int m = 0; m < width; ++m) {
            uint8_t d[5];
            uint32_t v;
            digits(src[start + m], d, &v);
            if ((v * 256 + 242) / 243 != src[start + m]) return false;
            for (int n = 0; n < 5; ++n) {
                const int index = position + n * width + m;
                dst[2 + index / 4] |= static_cast<uint8_t>(d[n] << (2 * (index % 4)));
            }
        }
        position += width * 5;
    }
    for (int h = 0; h < 2; ++h) {
        uint8_t d[5];
        uint32_t v;
        digits(src[24 + h], d, &v);
        if ((v / 3 * 3 * 256 + 242) / 243 != src[24 + h]) return false;
        for (int n = 0; n < 4; ++n) {
            const int index = 120 + n * 2 + h;
            dst[2 + index / 4] |= static_cast<uint8_t>(d[n] << (2 * (index % 4)));
        }
    }
    return true;
}

// ---- SHA-256 (FIPS 180-4), for the export receipt ---------------------------------------
struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint8_t buf[64];
    uint64_t len = 0;
    size_t fill = 0;
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void block(const uint8_t *p) {
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
        for (int t = 0; t < 16; ++t)
            w[t] = (uint32_t(p[4 * t]) << 24) | (uint32_t(p[4 * t + 1]) << 16) | (uint32_t(p[4 * t + 2]) << 8) |
                   p[4 * t + 3];
        for (int t = 16; t < 64; ++t) {
            const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int t = 0; t < 64; ++t) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K[t] + w[t];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    void update(const uint8_t *p, size_t n) {
        len += n;
        while (n) {
            const size_t take = n < 64 - fill ? n : 64 - fill;
            std::memcpy(buf + fill, p, take);
            fill += take;
            p += take;
            n -= take;
            if (fill == 64) {
                block(buf);
                fill = 0;
            }
        }
    }
    std::string hex() {
        const uint64_t bits = len * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t l[8];
        for (int k = 0; k < 8; ++k) l[k] = static_cast<uint8_t>(bits >> (56 - 8 * k));
        update(l, 8);
        char out[65];
        for (int k = 0; k < 8; ++k) std::snprintf(out + 8 * k, 9, "%08x", h[k]);
        return std::string(out, 64);
    }
};

}  // namespace

extern "C" {

void prism_gguf_default_policy(prism_gguf_policy *p) {
    if (!p) return;
    std::memset(p, 0, sizeof(*p));
    // IndexPolicy::new (tools/gguf/src/stream.rs:104-131)
    p->allow_zero_metadata = 1;
    p->max_file_bytes = 16ull << 30;
    p->max_tensors = 131072;
    p->max_metadata = 131072;
    p->metadata_budget = 128ull << 20;
    p->max_key_bytes = 65536;
    p->max_string_bytes = 16ull << 20;
    p->max_array_string_bytes = 16ull << 20;
    p->max_retained_string_array_bytes = 64ull << 20;
    p->max_array_items = 1000000;
    p->max_alignment = 1048576;
    p->reject_nonfinite_floats = 1;
    p->reject_interior_nul_keys = 1;
    p->reject_interior_nul_strings = 1;
    p->retain_string_arrays = 1;
}

int prism_gguf_open(const char *path, const prism_gguf_policy *policy, prism_gguf **out) {
    if (!path || !out) return bad(nullptr, "GGUF: null argument");
    *out = nullptr;
    prism_gguf_policy p;
    if (policy)
        p = *policy;
    else
        prism_gguf_default_policy(&p);
    struct stat st;
    if (stat(path, &st) != 0 || !S_ISREG(st.st_mode)) return bad(nullptr, "GGUF: a regular input file is required");
    FILE *f = std::fopen(path, "rb");
    if (!f) return bad(nullptr, "GGUF: cannot open the file");
    prism_gguf *g = new (std::nothrow) prism_gguf;
    if (!g) {
        std::fclose(f);
        return PRISM_ERR_RESOURCE;
    }
    g->path = path;
    g->file_bytes = static_cast<uint64_t>(st.st_size);
    int rc;
    try {
        rc = parse(g, f, p);
    } catch (...) {
        rc = bad(g, "GGUF: out of memory");
    }
    std::fclose(f);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return PRISM_OK;
}

void prism_gguf_close(prism_gguf *g) { delete g; }

const char *prism_gguf_last_error(void) { return g_last_error.c_str(); }

int prism_gguf_summary(const prism_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                       uint64_t *tensor_count, uint64_t *metadata_count, uint64_t *remaining_budget) {
    if (!g) return PRISM_ERR_INVALID_INPUT;
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (tensor_count) *tensor_count = g->tensors.size();
    if (metadata_count) *metadata_count = g->metadata.size();
    if (remaining_budget) *remaining_budget = g->remaining_budget;
    return PRISM_OK;
}

int prism_gguf_tensor_at(const prism_gguf *g, uint64_t index, const char **name, prism_gguf_tensor *info) {
    if (!g || index >= g->tensor_names.size()) return PRISM_ERR_INVALID_INPUT;
    const std::string &n = *g->tensor_names[index];
    if (name) *name = n.c_str();
    if (info) fill_info(g->tensors.at(n), info);
    return PRISM_OK;
}

int prism_gguf_find_tensor(const prism_gguf *g, const char *name, prism_gguf_tensor *info) {
    const Tensor *t = tensor_of(g, name);
    if (!t) return PRISM_ERR_INVALID_INPUT;
    if (info) fill_info(*t, info);
    return PRISM_OK;
}

int prism_gguf_metadata_at(const prism_gguf *g, uint64_t index, const char **key, uint32_t *type_id,
                           uint32_t *element_type_id, uint64_t *count, int *retained) {
    if (!g || index >= g->metadata_keys.size()) return PRISM_ERR_INVALID_INPUT;
    const std::string &k = *g->metadata_keys[index];
    const Meta &m = g->metadata.at(k);
    if (key) *key = k.c_str();
    if (type_id) *type_id = m.type;
    if (element_type_id) *element_type_id = m.elem;
    if (count) *count = m.count;
    if (retained) *retained = m.type == 9 ? (m.retained ? 1 : 0) : 1;
    return PRISM_OK;
}

int prism_gguf_metadata_int(const prism_gguf *g, const char *key, int64_t *out) {
    if (!g || !key || !out) return PRISM_ERR_INVALID_INPUT;
    auto it = g->metadata.find(key);
    if (it == g->metadata.end()) return PRISM_ERR_INVALID_INPUT;
    const Meta &m = it->second;
    switch (m.type) {
    case 0: case 2: case 4: case 7: *out = static_cast<int64_t>(m.u); return PRISM_OK;
    case 10:
        if (m.u > static_cast<uint64_t>(INT64_MAX)) return PRISM_ERR_INVALID_INPUT;
        *out = static_cast<int64_t>(m.u);
        return PRISM_OK;
    case 1: case 3: case 5: case 11: *out = m.i; return PRISM_OK;
    default: return PRISM_ERR_INVALID_INPUT;
    }
}

int prism_gguf_metadata_float(const prism_gguf *g, const char *key, double *out) {
    if (!g || !key || !out) return PRISM_ERR_INVALID_INPUT;
    auto it = g->metadata.find(key);
    if (it == g->metadata.end() || (it->second.type != 6 && it->second.type != 12)) return PRISM_ERR_INVALID_INPUT;
    *out = it->second.f;
    return PRISM_OK;
}

int prism_gguf_metadata_string(const prism_gguf *g, const char *key, uint64_t element, const char **text,
                               uint64_t *len) {
    if (!g || !key || !text) return PRISM_ERR_INVALID_INPUT;
    auto it = g->metadata.find(key);
    if (it == g->metadata.end()) return PRISM_ERR_INVALID_INPUT;
    const Meta &m = it->second;
    const std::string *s = nullptr;
    if (m.type == 8 && element == 0)
        s = &m.s;
    else if (m.type == 9 && m.elem == 8 && m.retained && element < m.strings.size())
        s = &m.strings[element];
    if (!s) return PRISM_ERR_INVALID_INPUT;
    *text = s->c_str();
    if (len) *len = s->size();
    return PRISM_OK;
}

int prism_gguf_read_tensor(const prism_gguf *g, const char *name, void *dst, uint64_t dst_len) {
    const Tensor *t = tensor_of(g, name);
    if (!t || !dst || dst_len != t->bytes) return PRISM_ERR_INVALID_INPUT;
    FILE *f = std::fopen(g->path.c_str(), "rb");
    if (!f) return bad(nullptr, "GGUF: cannot reopen the file");
    struct stat st;
    const bool same = fstat(fileno(f), &st) == 0 && static_cast<uint64_t>(st.st_size) == g->file_bytes;
    const bool ok = same && read_at(f, t->offset, dst, t->bytes);
    std::fclose(f);
    return ok ? PRISM_OK : bad(nullptr, "GGUF: tensor read failed (file changed or truncated)");
}

prism_weight_id prism_hip_weight_from_gguf(prism_hip_ctx *ctx, const prism_gguf *g, const char *name, uint64_t key) {
    const Tensor *t = tensor_of(g, name);
    if (!ctx || !t) return PRISM_ERR_INVALID_INPUT;
    // GGML order: dims[0] = columns (the packed axis), dims[1] = rows; higher dims must be 1.
    if (t->ndims > 2 && (t->dims[2] != 1 || (t->ndims > 3 && t->dims[3] != 1))) return PRISM_ERR_UNSUPPORTED;
    const uint64_t cols = t->dims[0], rows = t->ndims > 1 ? t->dims[1] : 1;
    std::vector<uint8_t> host;
    try {
        host.resize(t->bytes);
    } catch (...) {
        return PRISM_ERR_RESOURCE;
    }
    const int rc = prism_gguf_read_tensor(g, name, host.data(), host.size());
    if (rc) return rc;
    return prism_hip_weight_acquire(ctx, key, t->type, cols, rows, host.data(), host.size());
}

// export (tools/gguf/src/export.rs:130-318): general.file_type UINT32 141/142 -> 143,
// every PQ2 tensor's type -> 143 and its payload repacked (34 -> 28 bytes per block,
// each block re-expanded and compared), other payloads copied verbatim, extents laid
// out again in offset order at the file's alignment.  Writes a new file only.
int prism_gguf_export_ptq1(const char *src_path, const char *dst_path, char *receipt, size_t receipt_len) {
    if (!src_path || !dst_path) return bad(nullptr, "export: null path");
    prism_gguf_policy p;
    prism_gguf_default_policy(&p);
    p.prism_dialect = 1;
    p.retain_string_arrays = 0;
    prism_gguf *g = nullptr;
    int rc = prism_gguf_open(src_path, &p, &g);
    if (rc) return rc;
    auto fail = [&](const char *what) {
        delete g;
        return bad(nullptr, what);
    };
    auto ft = g->metadata.find("general.file_type");
    if (ft == g->metadata.end() || ft->second.type != 4 || !(ft->second.u == 141 || ft->second.u == 142))
        return fail("export: requires a UINT32 Prism PQ2 general.file_type (141 or 142)");
    std::vector<std::pair<const std::string *, const Tensor *>> ordered;
    bool any_pq2 = false;
    for (auto &kv : g->tensors) {
        ordered.emplace_back(&kv.first, &kv.second);
        any_pq2 |= kv.second.type == 142;
    }
    if (!any_pq2) return fail("export: requires at least one PQ2 tensor");
    std::sort(ordered.begin(), ordered.end(),
              [](const auto &a, const auto &b) { return a.second->offset < b.second->offset; });
    const uint64_t a = g->alignment;
    std::vector<uint64_t> offsets;
    uint64_t extent = 0, blocks = 0, converted = 0;
    for (auto &e : ordered) {
        const Tensor &t = *e.second;
        const uint64_t off = (extent + a - 1) / a * a;
        offsets.push_back(off);
        uint64_t bytes = t.bytes;
        if (t.type == 142) {
            blocks += t.elements / 128;
            ++converted;
            bytes = t.elements / 128 * 28;
        }
        extent = off + bytes;
    }
    const uint64_t out_bytes = g->data_offset + (extent + a - 1) / a * a;
    FILE *src = std::fopen(src_path, "rb");
    if (!src) return fail("export: cannot reopen the source");
    FILE *dst = std::fopen(dst_path, "w+bx");  // create_new: never overwrite
    if (!dst) {
        std::fclose(src);
        return fail("export: cannot create the output (it must not exist)");
    }
    std::vector<uint8_t> buf(1 << 16);
    bool ok = true;
    auto copy = [&](uint64_t from, uint64_t n) {
        ok = ok && std::fseek(src, static_cast<long>(from), SEEK_SET) == 0;
        while (ok && n) {
            const size_t take = n < buf.size() ? n : buf.size();
            ok = std::fread(buf.data(), 1, take, src) == take && std::fwrite(buf.data(), 1, take, dst) == take;
            n -= take;
        }
    };
    auto pad_to = [&](uint64_t pos) {
        const long cur = std::ftell(dst);
        ok = ok && cur >= 0 && static_cast<uint64_t>(cur) <= pos;
        static const uint8_t zeros[4096] = {0};
        for (uint64_t left = ok ? pos - cur : 0; ok && left;) {
            const size_t take = left < sizeof(zeros) ? left : sizeof(zeros);
            ok = std::fwrite(zeros, 1, take, dst) == take;
            left -= take;
        }
    };
    auto put32 = [&](uint64_t pos, uint32_t v) {
        ok = ok && std::fseek(dst, static_cast<long>(pos), SEEK_SET) == 0 && std::fwrite(&v, 4, 1, dst) == 1;
    };
    auto put64 = [&](uint64_t v) { ok = ok && std::fwrite(&v, 8, 1, dst) == 1; };
    copy(0, g->data_offset);
    put32(ft->second.value_pos, 143);
    for (size_t k = 0; k < ordered.size(); ++k) {
        const Tensor &t = *ordered[k].second;
        put32(t.type_pos, t.type == 142 ? 143u : t.type);
        put64(offsets[k]);
    }
    ok = ok && std::fseek(dst, static_cast<long>(g->data_offset), SEEK_SET) == 0;
    bool exact = true;
    for (size_t k = 0; ok && k < ordered.size(); ++k) {
        const Tensor &t = *ordered[k].second;
        pad_to(g->data_offset + offsets[k]);
        if (t.type != 142) {
            const long here = std::ftell(dst);
            copy(t.offset, t.bytes);
            ok = ok && std::fseek(dst, here + static_cast<long>(t.bytes), SEEK_SET) == 0;
            continue;
        }
        ok = ok && std::fseek(src, static_cast<long>(t.offset), SEEK_SET) == 0;
        uint8_t in[34], outb[28], back[34];
        for (uint64_t b = 0; ok && b < t.elements / 128; ++b) {
            ok = std::fread(in, 1, 34, src) == 34;
            if (ok && !pack_ptq(in, outb)) {
                exact = false;
                ok = false;
                break;
            }
            exact = exact && unpack_ptq(outb, back) && std::memcmp(back, in, 34) == 0;
            ok = ok && exact && std::fwrite(outb, 1, 28, dst) == 28;
        }
    }
    pad_to(out_bytes);
    ok = ok && std::fflush(dst) == 0;
    std::string sha;
    if (ok) {
        Sha256 h;
        ok = std::fseek(dst, 0, SEEK_SET) == 0;
        for (uint64_t left = out_bytes; ok && left;) {
            const size_t take = left < buf.size() ? left : buf.size();
            ok = std::fread(buf.data(), 1, take, dst) == take;
            h.update(buf.data(), take);
            left -= take;
        }
        sha = h.hex();
    }
    std::fclose(src);
    std::fclose(dst);
    const uint64_t src_bytes = g->file_bytes;
    delete g;
    if (!exact) return bad(nullptr, "export: a PQ2 block has no exact PTQ1 form (code 3 or unusable scale)");
    if (!ok) return bad(nullptr, "export: I/O failure");
    if (receipt && receipt_len) {
        std::snprintf(receipt, receipt_len,
                      "{\"SchemaVersion\":1,\"SourceBytes\":%llu,\"OutputBytes\":%llu,\"OutputSha256\":\"%s\","
                      "\"ConvertedTensorCount\":%llu,\"ConvertedBlocks\":%llu,"
                      "\"ExactPq2ReconstructionVerified\":true,\"NonPq2TensorBytesCopiedVerbatim\":true}",
                      static_cast<unsigned long long>(src_bytes), static_cast<unsigned long long>(out_bytes),
                      sha.c_str(), static_cast<unsigned long long>(converted), static_cast<unsigned long long>(blocks));
    }
    return PRISM_OK;
}

}  // extern "C"
