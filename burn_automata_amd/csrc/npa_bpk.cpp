// npa_bpk.cpp - the .bpk model container and its JSON manifest (host code).
//
// Container (crates/burn_automata/src/import.rs:16-18, 444-498): the 8-byte magic "BAUTBPK1", a
// little-endian u32 container version (1), a little-endian u64 payload length, the SHA-256 digest
// of the payload (32 bytes), then the payload: the JSON of BpkModelManifest (import.rs:20-31) with
// NpaConfig (crates/burn_automata/src/config.rs:30-53), HashGridConfig
// (crates/burn_automata_kernels/src/config.rs:20-29), NpaWeights (model.rs:12-17) and an optional
// particle initialization (import.rs:33-71). load_manifest_bytes (import.rs:383-390) takes either
// a container or the bare JSON.
//
// The JSON reader follows serde_json's rules for these types: unknown fields are skipped, fields
// with a serde default may be absent, Option fields may be absent or null, integers (usize / u32)
// must be written as integer literals, f32 values are read as f64 and rounded to f32, enums with
// unit variants are their variant name as a string.
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/npa_abi.h"

namespace {

// ------------------------------------------------------------------ SHA-256 (FIPS 180-4)
struct Sha256 {
    uint32_t h[8];
    uint64_t bytes = 0;
    uint8_t block[64];
    size_t fill = 0;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    Sha256() {
        static const uint32_t init[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                         0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
        std::memcpy(h, init, sizeof(h));
    }

    void compress(const uint8_t* p) {
        static const uint32_t k[64] = {
            0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
            0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
            0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
            0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
            0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
            0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
            0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
            0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
        uint32_t w[64];
        for (int t = 0; t < 16; ++t)
            w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
        for (int t = 16; t < 64; ++t) {
            const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int t = 0; t < 64; ++t) {
            const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = hh + S1 + ch + k[t] + w[t];
            const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
            const uint32_t t2 = S0 + maj;
            hh = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h[0] += a;
        h[1] += b;
        h[2] += c;
        h[3] += d;
        h[4] += e;
        h[5] += f;
        h[6] += g;
        h[7] += hh;
    }

    void update(const uint8_t* p, size_t n) {
        bytes += n;
        while (n) {
            const size_t take = std::min<size_t>(n, 64 - fill);
            std::memcpy(block + fill, p, take);
            fill += take;
            p += take;
            n -= take;
            if (fill == 64) {
                compress(block);
                fill = 0;
            }
        }
    }

    void finish(uint8_t out[32]) {
        const uint64_t bits = bytes * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len, 8);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
    }
};

// ------------------------------------------------------------------ JSON reader
struct JsonError {
    std::string msg;
};

class Json {
  public:
    Json(const char* p, size_t n) : p_(p), end_(p + n), begin_(p) {}

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    [[noreturn]] void fail(const std::string& what) const {
        throw JsonError{what + " at byte " + std::to_string(p_ - begin_)};
    }
    bool peek(char c) {
        ws();
        return p_ < end_ && *p_ == c;
    }
    void expect(char c) {
        ws();
        if (p_ >= end_ || *p_ != c) fail(std::string("expected `") + c + "`");
        ++p_;
    }
    bool eat(char c) {
        if (!peek(c)) return false;
        ++p_;
        return true;
    }
    void end_of_input() {
        ws();
        if (p_ != end_) fail("trailing characters");
    }
    bool null_literal() { return literal("null"); }

    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (p_ >= end_) fail("EOF while parsing a string");
            const char c = *p_++;
            if (c == '"') return out;
            if ((unsigned char)c < 0x20) fail("control character in string");
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p_ >= end_) fail("EOF while parsing a string");
            const char e = *p_++;
            switch (e) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') fail("unpaired surrogate");
                        p_ += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) fail("invalid surrogate");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(cp, out);
                    break;
                }
                default: fail("invalid escape");
            }
        }
    }

    bool boolean() {
        if (literal("true")) return true;
        if (literal("false")) return false;
        fail("invalid type: expected a boolean");
    }

    // An integer literal (usize / u32 fields): no sign, fraction or exponent.
    uint64_t unsigned_integer() {
        const Number n = number();
        if (!n.integer || n.negative) fail("invalid type: expected an unsigned integer");
        uint64_t v = 0;
        auto r = std::from_chars(n.text, n.text + n.len, v);
        if (r.ec != std::errc() || r.ptr != n.text + n.len) fail("number out of range");
        return v;
    }

    // A usize field that this library's C ABI carries as u32 (dims, grid sizes): values above
    // u32::MAX are refused here rather than truncated.
    uint32_t u32_integer() {
        const uint64_t v = unsigned_integer();
        if (v > 0xFFFFFFFFull) fail("invalid value: integer out of range for u32");
        return (uint32_t)v;
    }

    // f32 field: the literal read as f64, then rounded to f32.
    float f32() {
        const Number n = number();
        double v = 0.0;
        auto r = std::from_chars(n.text, n.text + n.len, v);
        if (r.ec != std::errc() || r.ptr != n.text + n.len) fail("invalid number");
        return (float)v;
    }

    void f32_array(std::vector<float>& out) {
        out.clear();
        expect('[');
        if (eat(']')) return;
        do out.push_back(f32());
        while (eat(','));
        expect(']');
    }

    // Skips any value (unknown fields).
    void skip() {
        ws();
        if (p_ >= end_) fail("EOF while parsing a value");
        const char c = *p_;
        if (c == '{') {
            ++p_;
            if (eat('}')) return;
            do {
                string();
                expect(':');
                skip();
            } while (eat(','));
            expect('}');
        } else if (c == '[') {
            ++p_;
            if (eat(']')) return;
            do skip();
            while (eat(','));
            expect(']');
        } else if (c == '"') {
            string();
        } else if (c == 't' || c == 'f') {
            boolean();
        } else if (c == 'n') {
            if (!null_literal()) fail("expected value");
        } else {
            number();
        }
    }

    // Object fields: calls field(key) for each; field must consume the value.
    template <class F>
    void object(F&& field) {
        expect('{');
        if (eat('}')) return;
        do {
            const std::string key = string();
            expect(':');
            field(key);
        } while (eat(','));
        expect('}');
    }

  private:
    struct Number {
        const char* text;
        size_t len;
        bool integer, negative;
    };
    const char* p_;
    const char* end_;
    const char* begin_;

    bool literal(const char* word) {
        ws();
        const size_t n = std::strlen(word);
        if ((size_t)(end_ - p_) >= n && std::memcmp(p_, word, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) fail("EOF in \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else fail("invalid \\u escape");
        }
        return v;
    }
    static void utf8(uint32_t cp, std::string& out) {
        if (cp < 0x80) {
            out.push_back((char)cp);
        } else if (cp < 0x800) {
            out.push_back((char)(0xC0 | (cp >> 6)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
        } else if (cp < 0x10000) {
            out.push_back((char)(0xE0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
        } else {
            out.push_back((char)(0xF0 | (cp >> 18)));
            out.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
        }
    }
    // JSON number grammar: -?(0|[1-9][0-9]*)(.[0-9]+)?([eE][+-]?[0-9]+)?
    Number number() {
        ws();
        const char* s = p_;
        bool integer = true, negative = false;
        if (p_ < end_ && *p_ == '-') {
            negative = true;
            ++p_;
        }
        if (p_ >= end_ || !isdigit(*p_)) fail("invalid number");
        if (*p_ == '0') ++p_;
        else
            while (p_ < end_ && isdigit(*p_)) ++p_;
        if (p_ < end_ && *p_ == '.') {
            integer = false;
            ++p_;
            if (p_ >= end_ || !isdigit(*p_)) fail("invalid number");
            while (p_ < end_ && isdigit(*p_)) ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integer = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || !isdigit(*p_)) fail("invalid number");
            while (p_ < end_ && isdigit(*p_)) ++p_;
        }
        // from_chars takes no leading '+' and reads the '-' itself
        return Number{s, (size_t)(p_ - s), integer, negative};
    }
    static bool isdigit(char c) { return c >= '0' && c <= '9'; }
};

}  // namespace

// ------------------------------------------------------------------ manifest
struct npa_manifest {
    uint32_t format_version = 0;
    std::string model_kind, source;
    bool has_source = false;
    // NpaConfig
    uint64_t spatial_dims = 0, state_dims = 0, hidden_dims = 0, auxiliary_input_dims = 0;
    float eps0 = 0.0f, alpha = 0.0f;
    bool density_grad = false, state_grad = false, log_norm_grad = false, log_norm_density_grad = false;
    bool stopgrad_pos = false, stopgrad_state = false, position_features = false;
    uint32_t equivariance = NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE;
    bool has_decoder_dims = false, has_output_dims = false;
    uint64_t decoder_dims = 0, output_dims = 0;
    // HashGridConfig
    npa_grid_cfg grid{};
    uint64_t grid_dim = 0, grid_size[3] = {0, 0, 0}, max_particles_per_block = 0;
    // NpaWeights
    std::vector<float> w1, b1, w2, b2;
    // NpaParticleInitialization
    bool has_init = false;
    std::vector<float> init_positions, init_states;
};

namespace {

struct Required {
    std::vector<std::string> names;
    std::vector<bool> seen;
    explicit Required(std::initializer_list<const char*> n) {
        for (const char* s : n) names.emplace_back(s);
        seen.assign(names.size(), false);
    }
    void mark(Json& js, const std::string& k) {
        for (size_t i = 0; i < names.size(); ++i)
            if (names[i] == k) {
                if (seen[i]) js.fail("duplicate field `" + k + "`");
                seen[i] = true;
            }
    }
    void check(Json& js) const {
        for (size_t i = 0; i < names.size(); ++i)
            if (!seen[i]) js.fail("missing field `" + names[i] + "`");
    }
};

uint32_t enum_variant(Json& js, std::initializer_list<const char*> variants) {
    const std::string v = js.string();
    uint32_t i = 0;
    for (const char* s : variants) {
        if (v == s) return i;
        ++i;
    }
    js.fail("unknown variant `" + v + "`");
}

void read_config(Json& js, npa_manifest& m) {
    Required req({"spatial_dims", "state_dims", "hidden_dims", "eps0", "alpha", "density_grad", "state_grad",
                  "log_norm_grad", "log_norm_density_grad", "stopgrad_pos", "stopgrad_state"});
    js.object([&](const std::string& k) {
        req.mark(js, k);
        if (k == "spatial_dims") m.spatial_dims = js.u32_integer();
        else if (k == "state_dims") m.state_dims = js.u32_integer();
        else if (k == "hidden_dims") m.hidden_dims = js.u32_integer();
        else if (k == "eps0") m.eps0 = js.f32();
        else if (k == "alpha") m.alpha = js.f32();
        else if (k == "density_grad") m.density_grad = js.boolean();
        else if (k == "state_grad") m.state_grad = js.boolean();
        else if (k == "log_norm_grad") m.log_norm_grad = js.boolean();
        else if (k == "log_norm_density_grad") m.log_norm_density_grad = js.boolean();
        else if (k == "stopgrad_pos") m.stopgrad_pos = js.boolean();
        else if (k == "stopgrad_state") m.stopgrad_state = js.boolean();
        else if (k == "equivariance")  // EquivarianceMode config.rs:22-28
            m.equivariance = enum_variant(js, {"None", "ParticleDensity", "ParticleDensityAndScale"});
        else if (k == "position_features") m.position_features = js.boolean();
        else if (k == "auxiliary_input_dims") m.auxiliary_input_dims = js.u32_integer();
        else if (k == "decoder_dims") {
            m.has_decoder_dims = !js.null_literal();
            if (m.has_decoder_dims) m.decoder_dims = js.unsigned_integer();
        } else if (k == "output_dims") {
            m.has_output_dims = !js.null_literal();
            if (m.has_output_dims) m.output_dims = js.unsigned_integer();
        } else js.skip();
    });
    req.check(js);
}

void read_hashgrid(Json& js, npa_manifest& m) {
    Required req({"dim", "boundary", "mode", "grid_size", "eps", "max_particles_per_block"});
    js.object([&](const std::string& k) {
        req.mark(js, k);
        if (k == "dim") m.grid_dim = js.u32_integer();
        else if (k == "boundary") m.grid.boundary = enum_variant(js, {"Periodic", "Clamped"}) == 0 ? NPA_BOUNDARY_PERIODIC
                                                                                               : NPA_BOUNDARY_CLAMPED;
        else if (k == "mode") m.grid.mode = enum_variant(js, {"Grid", "Particle"}) == 0 ? NPA_MODE_GRID : NPA_MODE_PARTICLE;
        else if (k == "grid_size") {
            js.expect('[');
            for (int a = 0; a < 3; ++a) {
                if (a) js.expect(',');
                m.grid_size[a] = js.u32_integer();
            }
            if (!js.eat(']')) js.fail("invalid length, expected an array of length 3");
        } else if (k == "eps") m.grid.eps = js.f32();
        else if (k == "max_particles_per_block") m.max_particles_per_block = js.u32_integer();
        else js.skip();
    });
    req.check(js);
}

void read_weights(Json& js, npa_manifest& m) {
    Required req({"w1", "b1", "w2", "b2"});
    js.object([&](const std::string& k) {
        req.mark(js, k);
        if (k == "w1") js.f32_array(m.w1);
        else if (k == "b1") js.f32_array(m.b1);
        else if (k == "w2") js.f32_array(m.w2);
        else if (k == "b2") js.f32_array(m.b2);
        else js.skip();
    });
    req.check(js);
}

void read_initialization(Json& js, npa_manifest& m) {
    Required req({"positions", "states"});
    js.object([&](const std::string& k) {
        req.mark(js, k);
        if (k == "positions") {  // Vec<[f32; 4]>
            m.init_positions.clear();
            js.expect('[');
            if (!js.eat(']')) {
                do {
                    js.expect('[');
                    for (int a = 0; a < 4; ++a) {
                        if (a) js.expect(',');
                        m.init_positions.push_back(js.f32());
                    }
                    if (!js.eat(']')) js.fail("invalid length, expected an array of length 4");
                } while (js.eat(','));
                js.expect(']');
            }
        } else if (k == "states") js.f32_array(m.init_states);
        else js.skip();
    });
    req.check(js);
}

void read_manifest(Json& js, npa_manifest& m) {
    Required req({"format_version", "model_kind", "config", "hashgrid", "weights"});
    js.object([&](const std::string& k) {
        req.mark(js, k);
        if (k == "format_version") {
            const uint64_t v = js.unsigned_integer();
            if (v > 0xFFFFFFFFull) js.fail("invalid value: integer out of range for u32");
            m.format_version = (uint32_t)v;
        } else if (k == "model_kind") m.model_kind = js.string();
        else if (k == "source") {
            m.has_source = !js.null_literal();
            if (m.has_source) m.source = js.string();
        } else if (k == "config") read_config(js, m);
        else if (k == "hashgrid") read_hashgrid(js, m);
        else if (k == "weights") read_weights(js, m);
        else if (k == "initialization") {
            m.has_init = !js.null_literal();
            if (m.has_init) read_initialization(js, m);
        } else js.skip();
    });
    req.check(js);
    js.end_of_input();
}

uint64_t perception_dims(const npa_manifest& m) {  // NpaConfig::perception_dims config.rs:133-139
    return m.state_dims * 2 + (m.state_grad ? m.state_dims * m.spatial_dims : 0) +
           (m.density_grad ? m.spatial_dims : 0) + (m.position_features ? m.spatial_dims : 0) +
           m.auxiliary_input_dims;
}

// validate_manifest import.rs:500-506: NpaModel::validate (model.rs:757-765, NpaWeights::validate
// model.rs:77-107), then NpaParticleInitialization::validate (import.rs:39-65).
npa_status validate(const npa_manifest& m, std::string* err) {
    if (!(m.spatial_dims == 2 || m.spatial_dims == 3)) {
        *err = "invalid model: spatial_dims must be 2 or 3, got " + std::to_string(m.spatial_dims);
        return NPA_ERR_INVALID_MODEL;
    }
    const uint64_t F = perception_dims(m), H = m.hidden_dims, O = m.spatial_dims + m.state_dims;
    const struct {
        const char* name;
        uint64_t got, want;
    } lens[] = {{"w1", m.w1.size(), H * F}, {"b1", m.b1.size(), H}, {"w2", m.w2.size(), O * H}, {"b2", m.b2.size(), O}};
    for (const auto& l : lens)
        if (l.got != l.want) {
            *err = std::string("invalid model: ") + l.name + " len " + std::to_string(l.got) + " != " +
                   std::to_string(l.want);
            return NPA_ERR_INVALID_MODEL;
        }
    if (m.has_init) {
        const uint64_t n = m.init_positions.size() / 4;
        if (n == 0) {
            *err = "invalid model: particle initialization cannot be empty";
            return NPA_ERR_INVALID_MODEL;
        }
        if (m.init_states.size() != n * m.state_dims) {
            *err = "invalid model: particle initialization has " + std::to_string(m.init_states.size()) +
                   " state values; expected " + std::to_string(n) + " positions * " + std::to_string(m.state_dims) +
                   " state dims";
            return NPA_ERR_INVALID_MODEL;
        }
        for (float v : m.init_positions)
            if (!std::isfinite(v)) {
                *err = "invalid model: particle initialization contains non-finite values";
                return NPA_ERR_INVALID_MODEL;
            }
        for (float v : m.init_states)
            if (!std::isfinite(v)) {
                *err = "invalid model: particle initialization contains non-finite values";
                return NPA_ERR_INVALID_MODEL;
            }
    }
    return NPA_OK;
}

constexpr uint8_t kMagic[8] = {'B', 'A', 'U', 'T', 'B', 'P', 'K', '1'};
constexpr size_t kHeaderLen = 8 + 4 + 8 + 32;
constexpr uint32_t kContainerVersion = 1;

void set_err(char* buf, size_t len, const std::string& msg) {
    if (!buf || !len) return;
    const size_t n = std::min(len - 1, msg.size());
    std::memcpy(buf, msg.data(), n);
    buf[n] = 0;
}

uint64_t le64(const uint8_t* p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = v << 8 | p[i];
    return v;
}

// decode_bpk_manifest import.rs:460-498 / load_manifest_bytes import.rs:383-390
npa_status load(const uint8_t* bytes, size_t len, npa_manifest* m, std::string* err) {
    const uint8_t* payload = bytes;
    size_t plen = len;
    if (len >= 8 && std::memcmp(bytes, kMagic, 8) == 0) {
        if (len < kHeaderLen) {
            *err = "invalid model format: bpk file is shorter than header: " + std::to_string(len) + " < " +
                   std::to_string(kHeaderLen);
            return NPA_ERR_INVALID_FORMAT;
        }
        const uint32_t version = (uint32_t)bytes[8] | (uint32_t)bytes[9] << 8 | (uint32_t)bytes[10] << 16 |
                                 (uint32_t)bytes[11] << 24;
        if (version != kContainerVersion) {
            *err = "invalid model format: unsupported bpk container version " + std::to_string(version);
            return NPA_ERR_INVALID_FORMAT;
        }
        const uint64_t payload_len = le64(bytes + 12);
        const uint64_t expected = kHeaderLen + payload_len;
        if (payload_len > len || (uint64_t)len != expected) {
            *err = "invalid model format: bpk payload length mismatch: file " + std::to_string(len) +
                   " != expected " + std::to_string(expected);
            return NPA_ERR_INVALID_FORMAT;
        }
        payload = bytes + kHeaderLen;
        plen = (size_t)payload_len;
        uint8_t digest[32];
        Sha256 sh;
        sh.update(payload, plen);
        sh.finish(digest);
        if (std::memcmp(digest, bytes + 20, 32) != 0) {
            *err = "invalid model format: bpk sha256 checksum mismatch";
            return NPA_ERR_INVALID_FORMAT;
        }
    }
    try {
        Json js(reinterpret_cast<const char*>(payload), plen);
        read_manifest(js, *m);
    } catch (const JsonError& e) {
        *err = e.msg;
        return NPA_ERR_JSON;
    }
    m->grid.dim = (uint32_t)m->grid_dim;
    for (int a = 0; a < 3; ++a) m->grid.grid_size[a] = (uint32_t)m->grid_size[a];
    m->grid.max_particles_per_block = (uint32_t)m->max_particles_per_block;
    return validate(*m, err);
}

}  // namespace

extern "C" {

npa_status npa_manifest_load(const uint8_t* bytes, size_t len, npa_manifest** out, char* err, size_t err_len) {
    if (!out || (!bytes && len)) return NPA_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    npa_manifest* m = new (std::nothrow) npa_manifest();
    if (!m) return NPA_ERR_OUT_OF_MEMORY;
    std::string msg;
    npa_status st;
    try {
        st = load(bytes, len, m, &msg);
    } catch (const std::bad_alloc&) {
        st = NPA_ERR_OUT_OF_MEMORY;
        msg = "out of memory";
    }
    if (st != NPA_OK) {
        set_err(err, err_len, msg);
        delete m;
        return st;
    }
    set_err(err, err_len, "");
    *out = m;
    return NPA_OK;
}

npa_status npa_manifest_load_file(const char* path, npa_manifest** out, char* err, size_t err_len) {
    if (!path || !out) return NPA_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    FILE* f = std::fopen(path, "rb");
    if (!f) {
        set_err(err, err_len, std::string("cannot open ") + path + ": " + std::strerror(errno));
        return NPA_ERR_IO;
    }
    std::vector<uint8_t> buf;
    uint8_t chunk[1 << 16];
    size_t n;
    while ((n = std::fread(chunk, 1, sizeof(chunk), f)) > 0) buf.insert(buf.end(), chunk, chunk + n);
    const bool bad = std::ferror(f) != 0;
    std::fclose(f);
    if (bad) {
        set_err(err, err_len, std::string("cannot read ") + path);
        return NPA_ERR_IO;
    }
    return npa_manifest_load(buf.data(), buf.size(), out, err, err_len);
}

void npa_manifest_destroy(npa_manifest* m) { delete m; }

npa_status npa_manifest_info(const npa_manifest* m, npa_manifest_info_t* info) {
    if (!m || !info) return NPA_ERR_INVALID_ARGUMENT;
    info->format_version = m->format_version;
    info->model_kind = m->model_kind.c_str();
    info->source = m->has_source ? m->source.c_str() : nullptr;
    info->auxiliary_input_dims = (uint32_t)m->auxiliary_input_dims;
    info->decoder_dims = m->has_decoder_dims ? (int64_t)m->decoder_dims : -1;
    info->output_dims = m->has_output_dims ? (int64_t)m->output_dims : -1;
    info->stopgrad_pos = m->stopgrad_pos;
    info->stopgrad_state = m->stopgrad_state;
    info->initialization_particles = m->has_init ? (uint32_t)(m->init_positions.size() / 4) : 0;
    return NPA_OK;
}

npa_status npa_manifest_model(const npa_manifest* m, npa_model_cfg* model, npa_grid_cfg* grid, npa_weights* weights) {
    if (!m) return NPA_ERR_INVALID_ARGUMENT;
    if (m->auxiliary_input_dims != 0) return NPA_ERR_INVALID_MODEL;  // no auxiliary rows on the device path
    if (model) {
        model->spatial_dims = (uint32_t)m->spatial_dims;
        model->state_dims = (uint32_t)m->state_dims;
        model->hidden_dims = (uint32_t)m->hidden_dims;
        model->eps0 = m->eps0;
        model->alpha = m->alpha;
        model->density_grad = m->density_grad;
        model->state_grad = m->state_grad;
        model->log_norm_grad = m->log_norm_grad;
        model->log_norm_density_grad = m->log_norm_density_grad;
        model->equivariance = m->equivariance;
        model->position_features = m->position_features;
    }
    if (grid) *grid = m->grid;
    if (weights) {
        weights->w1 = m->w1.data();
        weights->b1 = m->b1.data();
        weights->w2 = m->w2.data();
        weights->b2 = m->b2.data();
    }
    return NPA_OK;
}

npa_status npa_manifest_initialization(const npa_manifest* m, const float** positions, const float** states,
                                       uint32_t* particle_count) {
    if (!m) return NPA_ERR_INVALID_ARGUMENT;
    if (!m->has_init) return NPA_ERR_INVALID_ARGUMENT;
    if (positions) *positions = m->init_positions.data();
    if (states) *states = m->init_states.data();
    if (particle_count) *particle_count = (uint32_t)(m->init_positions.size() / 4);
    return NPA_OK;
}

npa_status npa_bpk_encode(const uint8_t* payload, size_t len, uint8_t* out, size_t out_len, size_t* required) {
    if (!payload && len) return NPA_ERR_INVALID_ARGUMENT;
    const size_t need = kHeaderLen + len;
    if (required) *required = need;
    if (!out) return NPA_OK;
    if (out_len < need) return NPA_ERR_OUTPUT_SHAPE;
    std::memcpy(out, kMagic, 8);
    for (int i = 0; i < 4; ++i) out[8 + i] = (uint8_t)(kContainerVersion >> (8 * i));
    for (int i = 0; i < 8; ++i) out[12 + i] = (uint8_t)((uint64_t)len >> (8 * i));
    Sha256 sh;
    sh.update(payload, len);
    sh.finish(out + 20);
    if (len) std::memcpy(out + kHeaderLen, payload, len);
    return NPA_OK;
}

npa_status npa_sha256(const uint8_t* data, size_t len, uint8_t* digest) {
    if ((!data && len) || !digest) return NPA_ERR_INVALID_ARGUMENT;
    Sha256 sh;
    sh.update(data, len);
    sh.finish(digest);
    return NPA_OK;
}

}  // extern "C"
