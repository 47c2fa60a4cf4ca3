// safetensors.cpp — see safetensors.hpp.
#include "safetensors.hpp"

#include <cctype>
#include <cerrno>
#include <cstring>
#include <fstream>
#include <limits>
#include <optional>
#include <sstream>

#include <stdlib.h>
#include <unistd.h>

namespace soklyn {

namespace {

[[noreturn]] void fail(ErrorKind kind, const std::string &what) { throw Error(kind, host_status(kind), what); }

// ---- JSON -------------------------------------------------------------------------------------
struct Parser {
    const std::string &s;
    size_t i = 0;

    [[noreturn]] void err(const std::string &m) {
        fail(ErrorKind::SerdeJSON, "JSON error: " + m + " at byte " + std::to_string(i));
    }
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) ++i;
    }
    bool lit(const char *w) {
        const size_t n = std::strlen(w);
        if (s.compare(i, n, w) != 0) return false;
        i += n;
        return true;
    }
    static void utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xc0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xe0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
            out += static_cast<char>(0x80 | (cp & 0x3f));
        } else {
            out += static_cast<char>(0xf0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3f));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
            out += static_cast<char>(0x80 | (cp & 0x3f));
        }
    }
    uint32_t hex4() {
        if (i + 4 > s.size()) err("EOF while parsing a string");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s[i++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else err("invalid escape");
        }
        return v;
    }
    std::string str() {
        ++i;   // opening quote
        std::string out;
        while (true) {
            if (i >= s.size()) err("EOF while parsing a string");
            const unsigned char c = static_cast<unsigned char>(s[i++]);
            if (c == '"') return out;
            if (c < 0x20) err("control character in string");
            if (c != '\\') {
                out += static_cast<char>(c);
                continue;
            }
            if (i >= s.size()) err("EOF while parsing a string");
            const char e = s[i++];
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                uint32_t cp = hex4();
                if (cp >= 0xd800 && cp < 0xdc00) {
                    if (!lit("\\u")) err("lone leading surrogate");
                    const uint32_t lo = hex4();
                    if (lo < 0xdc00 || lo >= 0xe000) err("invalid trailing surrogate");
                    cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                } else if (cp >= 0xdc00 && cp < 0xe000) {
                    err("lone trailing surrogate");
                }
                utf8(out, cp);
                break;
            }
            default: err("invalid escape");
            }
        }
    }
    std::string number() {
        const size_t b = i;
        if (s[i] == '-') ++i;
        if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) err("invalid number");
        if (s[i] == '0') ++i;
        else while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
        if (i < s.size() && s[i] == '.') {
            ++i;
            if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) err("invalid number");
            while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
        }
        if (i < s.size() && (s[i] == 'e' || s[i] == 'E')) {
            ++i;
            if (i < s.size() && (s[i] == '+' || s[i] == '-')) ++i;
            if (i >= s.size() || !isdigit(static_cast<unsigned char>(s[i]))) err("invalid number");
            while (i < s.size() && isdigit(static_cast<unsigned char>(s[i]))) ++i;
        }
        return s.substr(b, i - b);
    }
    JsonValue value(int depth) {
        if (depth > 128) err("recursion limit exceeded");
        ws();
        if (i >= s.size()) err("EOF while parsing a value");
        JsonValue v;
        const char c = s[i];
        if (c == '{') {
            v.kind = JsonValue::Kind::Object;
            ++i;
            ws();
            if (i < s.size() && s[i] == '}') {
                ++i;
                return v;
            }
            while (true) {
                ws();
                if (i >= s.size() || s[i] != '"') err("key must be a string");
                std::string k = str();
                ws();
                if (i >= s.size() || s[i] != ':') err("expected `:`");
                ++i;
                v.members[k] = value(depth + 1);
                ws();
                if (i < s.size() && s[i] == ',') { ++i; continue; }
                if (i < s.size() && s[i] == '}') { ++i; return v; }
                err("expected `,` or `}`");
            }
        }
        if (c == '[') {
            v.kind = JsonValue::Kind::Array;
            ++i;
            ws();
            if (i < s.size() && s[i] == ']') {
                ++i;
                return v;
            }
            while (true) {
                v.items.push_back(value(depth + 1));
                ws();
                if (i < s.size() && s[i] == ',') { ++i; continue; }
                if (i < s.size() && s[i] == ']') { ++i; return v; }
                err("expected `,` or `]`");
            }
        }
        if (c == '"') {
            v.kind = JsonValue::Kind::String;
            v.text = str();
            return v;
        }
        if (lit("true")) { v.kind = JsonValue::Kind::Bool; v.text = "true"; return v; }
        if (lit("false")) { v.kind = JsonValue::Kind::Bool; v.text = "false"; return v; }
        if (lit("null")) return v;
        v.kind = JsonValue::Kind::Number;
        v.text = number();
        return v;
    }
};

// serde_json's escaping: \" \\ and the short escapes, other control bytes as \u00xx
void quote(std::string &out, const std::string &s) {
    static const char *hex = "0123456789abcdef";
    out += '"';
    for (unsigned char c : s) {
        switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\b': out += "\\b"; break;
        case '\f': out += "\\f"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
            if (c < 0x20) {
                out += "\\u00";
                out += hex[c >> 4];
                out += hex[c & 15];
            } else {
                out += static_cast<char>(c);
            }
        }
    }
    out += '"';
}

void emit(const JsonValue &v, std::string &out, int level, bool pretty) {
    auto nl = [&](int lv) {
        if (!pretty) return;
        out += '\n';
        out.append(static_cast<size_t>(2 * lv), ' ');
    };
    switch (v.kind) {
    case JsonValue::Kind::Null: out += "null"; return;
    case JsonValue::Kind::Bool:
    case JsonValue::Kind::Number: out += v.text; return;
    case JsonValue::Kind::String: quote(out, v.text); return;
    case JsonValue::Kind::Array: {
        if (v.items.empty()) {
            out += "[]";
            return;
        }
        out += '[';
        bool first = true;
        for (const JsonValue &it : v.items) {
            if (!first) out += ',';
            first = false;
            nl(level + 1);
            emit(it, out, level + 1, pretty);
        }
        nl(level);
        out += ']';
        return;
    }
    case JsonValue::Kind::Object: {
        if (v.members.empty()) {
            out += "{}";
            return;
        }
        out += '{';
        bool first = true;
        for (const auto &kv : v.members) {
            if (!first) out += ',';
            first = false;
            nl(level + 1);
            quote(out, kv.first);
            out += pretty ? ": " : ":";
            emit(kv.second, out, level + 1, pretty);
        }
        nl(level);
        out += '}';
        return;
    }
    }
}

JsonValue jstr(const std::string &s) {
    JsonValue v;
    v.kind = JsonValue::Kind::String;
    v.text = s;
    return v;
}
JsonValue jnum(size_t n) {
    JsonValue v;
    v.kind = JsonValue::Kind::Number;
    v.text = std::to_string(n);
    return v;
}

// serde's usize from a JSON number: a non-negative integer literal that fits
size_t as_usize(const JsonValue &v, const char *what) {
    if (v.kind != JsonValue::Kind::Number || v.text.empty() || v.text[0] == '-' ||
        v.text.find_first_of(".eE") != std::string::npos)
        fail(ErrorKind::SerdeJSON, std::string("JSON error: invalid type for ") + what + ", expected usize");
    errno = 0;
    char *end = nullptr;
    const unsigned long long x = std::strtoull(v.text.c_str(), &end, 10);
    if (errno || *end) fail(ErrorKind::SerdeJSON, std::string("JSON error: number out of range for ") + what);
    return static_cast<size_t>(x);
}

template <class U> std::vector<uint8_t> bytes_of(const std::vector<U> &v) {
    std::vector<uint8_t> b(v.size() * sizeof(U));
    if (!b.empty()) std::memcpy(b.data(), v.data(), b.size());
    return b;
}

// bytemuck::pod_collect_to_vec: ceil(len / size) elements, the tail zero-filled
template <class U> std::vector<U> collect(const std::vector<uint8_t> &b) {
    std::vector<U> v((b.size() + sizeof(U) - 1) / sizeof(U));
    if (!b.empty()) std::memcpy(v.data(), b.data(), b.size());
    return v;
}

}  // namespace

JsonValue JsonValue::parse(const std::string &src) {
    Parser p{src};
    JsonValue v = p.value(0);
    p.ws();
    if (p.i != src.size()) p.err("trailing characters");
    return v;
}
std::string JsonValue::to_pretty() const {
    std::string out;
    emit(*this, out, 0, true);
    return out;
}
std::string JsonValue::to_compact() const {
    std::string out;
    emit(*this, out, 0, false);
    return out;
}

// ---- SafetensorWriter (safetensor.rs) -------------------------------------------------------------
void SafetensorWriter::pass(std::string name, std::vector<size_t> shape, std::vector<uint8_t> data,
                            Precision precision) {
    descriptors_.push_back({std::move(name), std::move(shape), std::move(data), precision});
}

void SafetensorWriter::pass_metadata(const std::string &key, const std::string &value) {
    for (auto &kv : metadata_)
        if (kv.first == key) {
            kv.second = value;
            return;
        }
    metadata_.emplace_back(key, value);
}

// safetensor.rs:151-202
std::string SafetensorWriter::header_json() const {
    JsonValue top;
    top.kind = JsonValue::Kind::Object;
    if (!metadata_.empty()) {
        JsonValue m;
        m.kind = JsonValue::Kind::Object;
        for (const auto &kv : metadata_) m.members[kv.first] = jstr(kv.second);
        top.members["__metadata__"] = m;
    }
    size_t off = 0;
    for (const SafetensorDescriptor &d : descriptors_) {
        const size_t end = off + d.data.size();
        JsonValue desc;
        desc.kind = JsonValue::Kind::Object;
        desc.members["dtype"] = jstr(d.precision == Precision::FP32 ? "F32" : "F16");
        JsonValue shape, offs;
        shape.kind = offs.kind = JsonValue::Kind::Array;
        for (size_t x : d.shape) shape.items.push_back(jnum(x));
        offs.items = {jnum(off), jnum(end)};
        desc.members["shape"] = shape;
        desc.members["data_offsets"] = offs;
        top.members[d.name] = desc;
        off = end;
    }
    std::string json = top.to_pretty();
    if (json.size() % 8) json.append(8 - json.size() % 8, ' ');
    return json;
}

void SafetensorWriter::write(std::ostream &out) const {
    const std::string json = header_json();
    const uint64_t n = json.size();
    uint8_t le[8];
    for (int b = 0; b < 8; ++b) le[b] = static_cast<uint8_t>(n >> (8 * b));
    out.write(reinterpret_cast<const char *>(le), 8);
    out.write(json.data(), static_cast<std::streamsize>(json.size()));
    for (const SafetensorDescriptor &d : descriptors_)
        out.write(reinterpret_cast<const char *>(d.data.data()), static_cast<std::streamsize>(d.data.size()));
    out.flush();
    if (!out) fail(ErrorKind::IOError, "I/O error: writing safetensors data");
}

// safetensor.rs:77-136
SafetensorWriter SafetensorWriter::read(std::istream &in) {
    uint8_t le[8];
    if (!in.read(reinterpret_cast<char *>(le), 8)) fail(ErrorKind::IOError, "I/O error: failed to fill whole buffer");
    uint64_t n = 0;
    for (int b = 7; b >= 0; --b) n = (n << 8) | le[b];
    if (n > (uint64_t)1 << 40) fail(ErrorKind::TryFromIntError, "header size out of range");
    std::string header(static_cast<size_t>(n), '\0');
    if (n && !in.read(&header[0], static_cast<std::streamsize>(n)))
        fail(ErrorKind::IOError, "I/O error: failed to fill whole buffer");
    const JsonValue top = JsonValue::parse(header);
    if (top.kind != JsonValue::Kind::Object) fail(ErrorKind::SerdeJSON, "JSON error: invalid type, expected a map");
    const uint64_t base = 8 + n;
    SafetensorWriter w;
    for (const auto &kv : top.members) {
        const std::string &key = kv.first;
        const JsonValue &val = kv.second;
        if (key == "__metadata__") {
            if (val.kind == JsonValue::Kind::Object)
                for (const auto &m : val.members)
                    w.pass_metadata(m.first, m.second.kind == JsonValue::Kind::String ? m.second.text
                                                                                       : m.second.to_compact());
            continue;
        }
        if (val.kind != JsonValue::Kind::Object) fail(ErrorKind::SerdeJSON, "JSON error: invalid type for " + key);
        auto field = [&](const char *f) -> const JsonValue & {
            auto it = val.members.find(f);
            if (it == val.members.end()) fail(ErrorKind::SerdeJSON, std::string("JSON error: missing field `") + f + "`");
            return it->second;
        };
        const JsonValue &dt = field("dtype"), &sh = field("shape"), &of = field("data_offsets");
        if (dt.kind != JsonValue::Kind::String) fail(ErrorKind::SerdeJSON, "JSON error: invalid type for dtype");
        if (sh.kind != JsonValue::Kind::Array || of.kind != JsonValue::Kind::Array || of.items.size() != 2)
            fail(ErrorKind::SerdeJSON, "JSON error: invalid shape or data_offsets for " + key);
        if (dt.text != "F32" && dt.text != "F16")
            fail(ErrorKind::UnrecognizedTensorKey, "Unrecognized tensor key " + key + " with dtype \"" + dt.text + "\"");
        SafetensorDescriptor d;
        d.name = key;
        for (const JsonValue &x : sh.items) d.shape.push_back(as_usize(x, "shape"));
        const size_t o0 = as_usize(of.items[0], "data_offsets"), o1 = as_usize(of.items[1], "data_offsets");
        if (o1 < o0) fail(ErrorKind::IOError, "I/O error: invalid data offsets for " + key);
        d.data.resize(o1 - o0);
        in.clear();
        in.seekg(static_cast<std::streamoff>(base + o0));
        if (!d.data.empty() && !in.read(reinterpret_cast<char *>(d.data.data()), static_cast<std::streamsize>(d.data.size())))
            fail(ErrorKind::IOError, "I/O error: failed to fill whole buffer");
        d.precision = dt.text == "F16" ? Precision::FP16 : Precision::FP32;
        w.descriptors_.push_back(std::move(d));
    }
    return w;
}

// ---- SafetensorFile (save.rs) -------------------------------------------------------------------
template <class T>
SafetensorFile SafetensorFile::from_ffn(const GpuContext &ctx, const FeedForwardNetwork<T> &network) {
    return from_blocks(ctx, network.get_layers());
}

template <class T>
SafetensorFile SafetensorFile::from_blocks(const GpuContext &ctx, const std::vector<DenseBlock<T>> &blocks) {
    SafetensorFile f;
    f.pass_blocks(ctx, blocks);
    return f;
}

template <class T> void SafetensorFile::pass_blocks(const GpuContext &ctx, const std::vector<DenseBlock<T>> &blocks) {
    for (size_t i = 0; i < blocks.size(); ++i) pass_layer(ctx, blocks[i], i + 1);
}

template <class T> void SafetensorFile::pass_layer(const GpuContext &ctx, const DenseBlock<T> &layer, size_t layer_num) {
    const std::string pre = "layer" + std::to_string(layer_num) + ".";
    const Tensor2D<T> &w = layer.get_weights(), &b = layer.get_biases();
    const Tensor2D<T> &nw = layer.get_norm_weights(), &nb = layer.get_norm_biases();
    const std::vector<size_t> w_shape{w.rows(), w.cols()}, b_shape{b.cols()}, nw_shape{nw.cols()}, nb_shape{nb.cols()};
    const Precision tp = PrecisionType<T>::precision;
    writer_.pass(pre + "w", w_shape, bytes_of(w.download(ctx)), tp);
    writer_.pass(pre + "b", b_shape, bytes_of(b.download(ctx)), tp);
    writer_.pass(pre + "norm_w", nw_shape, bytes_of(nw.download(ctx)), tp);
    writer_.pass(pre + "norm_b", nb_shape, bytes_of(nb.download(ctx)), tp);
    if (!layer.is_training_mode()) return;
    const std::pair<const char *, std::pair<std::vector<size_t>, const Tensor2D<float> *>> moments[] = {
        {"dv_w", {w_shape, &layer.get_dv_weights()}},        {"dv_b", {b_shape, &layer.get_dv_biases()}},
        {"dm_w", {w_shape, &layer.get_dm_weights()}},        {"dm_b", {b_shape, &layer.get_dm_biases()}},
        {"dv_norm_w", {nw_shape, &layer.get_dv_norm_weights()}}, {"dv_norm_b", {nb_shape, &layer.get_dv_norm_biases()}},
        {"dm_norm_w", {nw_shape, &layer.get_dm_norm_weights()}}, {"dm_norm_b", {nb_shape, &layer.get_dm_norm_biases()}},
    };
    for (const auto &m : moments)
        writer_.pass(pre + m.first, m.second.first, bytes_of(m.second.second->download(ctx)), Precision::FP32);
    const std::pair<const char *, const std::optional<Tensor2D<float>> *> masters[] = {
        {"master_w", &layer.get_master_weights()},
        {"master_b", &layer.get_master_biases()},
        {"master_norm_w", &layer.get_master_norm_weights()},
        {"master_norm_b", &layer.get_master_norm_biases()},
    };
    for (const auto &m : masters)
        if (*m.second)
            writer_.pass(pre + m.first, {(*m.second)->rows(), (*m.second)->cols()}, bytes_of((*m.second)->download(ctx)),
                         Precision::FP32);
}

// save.rs:365-377: a temporary file in the target directory, persisted by rename
void SafetensorFile::save(const std::string &path) const {
    const size_t slash = path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? "." : (slash == 0 ? "/" : path.substr(0, slash));
    std::string tmpl = dir + "/.tmpXXXXXX";
    const int fd = mkstemp(&tmpl[0]);
    if (fd < 0) fail(ErrorKind::IOError, "I/O error: cannot create a temporary file in " + dir);
    close(fd);
    {
        std::ofstream out(tmpl, std::ios::binary | std::ios::trunc);
        try {
            if (!out) fail(ErrorKind::IOError, "I/O error: cannot open " + tmpl);
            writer_.write(out);
        } catch (...) {
            out.close();
            unlink(tmpl.c_str());
            throw;
        }
    }
    if (rename(tmpl.c_str(), path.c_str()) != 0) {
        unlink(tmpl.c_str());
        fail(ErrorKind::PersistError, "Temp file writing error: cannot persist to " + path);
    }
}

SafetensorFile SafetensorFile::read(const std::string &path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) fail(ErrorKind::IOError, "I/O error: cannot open " + path);
    SafetensorFile f;
    f.writer_ = SafetensorWriter::read(in);
    return f;
}

namespace {
enum class Param { W, B, MasterW, MasterB, NormW, NormB, MasterNormW, MasterNormB,
                   DvW, DvB, DmW, DmB, DvNormW, DvNormB, DmNormW, DmNormB, None };

// save.rs:40-97
Param param_from_str(const std::string &s) {
    static const std::pair<const char *, Param> names[] = {
        {"w", Param::W}, {"b", Param::B}, {"master_w", Param::MasterW}, {"master_b", Param::MasterB},
        {"norm_w", Param::NormW}, {"norm_b", Param::NormB}, {"master_norm_w", Param::MasterNormW},
        {"master_norm_b", Param::MasterNormB}, {"dv_w", Param::DvW}, {"dv_b", Param::DvB}, {"dm_w", Param::DmW},
        {"dm_b", Param::DmB}, {"dv_norm_w", Param::DvNormW}, {"dv_norm_b", Param::DvNormB},
        {"dm_norm_w", Param::DmNormW}, {"dm_norm_b", Param::DmNormB}};
    for (const auto &n : names)
        if (s == n.first) return n.second;
    return Param::None;
}
bool f32_only(Param p) { return p >= Param::MasterW && p != Param::NormW && p != Param::NormB; }
bool is_vector(Param p) {
    return p == Param::B || p == Param::DvB || p == Param::DmB || p == Param::NormW || p == Param::NormB ||
           p == Param::MasterNormW || p == Param::MasterNormB || p == Param::DvNormW || p == Param::DvNormB ||
           p == Param::DmNormW || p == Param::DmNormB;
}

// Rust's usize::from_str: an optional '+', then decimal digits, no overflow
bool parse_usize(const std::string &s, size_t &out) {
    size_t i = s.size() > 0 && s[0] == '+' ? 1 : 0;
    if (i >= s.size()) return false;
    unsigned long long v = 0;
    for (; i < s.size(); ++i) {
        if (s[i] < '0' || s[i] > '9') return false;
        const unsigned d = static_cast<unsigned>(s[i] - '0');
        if (v > (std::numeric_limits<unsigned long long>::max() - d) / 10) return false;
        v = v * 10 + d;
    }
    out = static_cast<size_t>(v);
    return true;
}

template <class U> struct HostMat {
    size_t rows = 0, cols = 0;
    std::vector<U> v;
};
template <class T> struct LayerParams {
    std::optional<HostMat<T>> w, b, norm_w, norm_b;
    std::optional<HostMat<float>> master_w, master_b, master_norm_w, master_norm_b;
    std::optional<HostMat<float>> dv_w, dv_b, dm_w, dm_b, dv_norm_w, dv_norm_b, dm_norm_w, dm_norm_b;
};
}  // namespace

template <class T>
std::vector<DenseBlock<T>> SafetensorFile::into_blocks(const GpuContext &ctx, bool is_training,
                                                       size_t max_batch_size) && {
    std::map<size_t, LayerParams<T>> layers;
    size_t max_layer = 0;
    for (const SafetensorDescriptor &d : writer_.get_descriptors()) {
        const std::string &name = d.name;
        if (name.compare(0, 5, "layer") != 0) continue;   // non-layer keys are skipped
        const std::string rest = name.substr(5);
        const size_t dot = rest.find('.');
        if (dot == std::string::npos)
            fail(ErrorKind::InvalidTensorName, "Invalid tensor name " + name + ": missing '.' separator");
        const std::string layer_str = rest.substr(0, dot), param_str = rest.substr(dot + 1);
        size_t idx = 0;
        if (!parse_usize(layer_str, idx))
            fail(ErrorKind::InvalidTensorName, "Invalid tensor name " + name + ": invalid layer index number");
        const Param p = param_from_str(param_str);
        if (p == Param::None)
            fail(ErrorKind::InvalidTensorName, "Invalid tensor name " + name + ": unrecognized parameter type");
        if (f32_only(p) && d.precision == Precision::FP16)
            fail(ErrorKind::PrecisionMatch,
                 "Layer " + layer_str + ": '" + param_str + "' must be FP32 but safetensor file contains FP16.");
        if (d.shape.size() < (is_vector(p) ? 1u : 2u))
            fail(ErrorKind::SerializationCasting, "tensor " + name + " has too few dimensions");
        const size_t rows = is_vector(p) ? 1 : d.shape[0], cols = is_vector(p) ? d.shape[0] : d.shape[1];
        LayerParams<T> &e = layers[idx];
        max_layer = idx > max_layer ? idx : max_layer;
        if (f32_only(p)) {
            HostMat<float> m{rows, cols, collect<float>(d.data)};
            switch (p) {
            case Param::MasterW: e.master_w = std::move(m); break;
            case Param::MasterB: e.master_b = std::move(m); break;
            case Param::MasterNormW: e.master_norm_w = std::move(m); break;
            case Param::MasterNormB: e.master_norm_b = std::move(m); break;
            default:
                if (!is_training) break;   // moments only in training mode
                switch (p) {
                case Param::DvW: e.dv_w = std::move(m); break;
                case Param::DvB: e.dv_b = std::move(m); break;
                case Param::DmW: e.dm_w = std::move(m); break;
                case Param::DmB: e.dm_b = std::move(m); break;
                case Param::DvNormW: e.dv_norm_w = std::move(m); break;
                case Param::DvNormB: e.dv_norm_b = std::move(m); break;
                case Param::DmNormW: e.dm_norm_w = std::move(m); break;
                case Param::DmNormB: e.dm_norm_b = std::move(m); break;
                default: break;
                }
            }
        } else {
            HostMat<T> m{rows, cols, collect<T>(d.data)};
            switch (p) {
            case Param::W: e.w = std::move(m); break;
            case Param::B: e.b = std::move(m); break;
            case Param::NormW: e.norm_w = std::move(m); break;
            case Param::NormB: e.norm_b = std::move(m); break;
            default: break;
            }
        }
    }
    if (max_layer == 0) fail(ErrorKind::NoLayersFound, "No network layers were found in safetensor file.");

    auto from_t = [&](const std::optional<HostMat<T>> &m, size_t r, size_t c) {
        return m ? Tensor2D<T>::from_cpu_vector(ctx, m->v, {r, c}) : Tensor2D<T>::zeros(ctx, {r, c});
    };
    auto from_f32 = [&](const std::optional<HostMat<float>> &m, size_t r, size_t c) -> std::optional<Tensor2D<float>> {
        if (!m) return std::nullopt;
        return Tensor2D<float>::from_cpu_vector(ctx, m->v, {r, c});
    };
    std::vector<DenseBlock<T>> blocks;
    for (size_t idx = 1; idx <= max_layer; ++idx) {
        auto it = layers.find(idx);
        if (it == layers.end())
            fail(ErrorKind::MissingLayer, "Layer " + std::to_string(idx) + " is completely missing from the safetensor file.");
        const LayerParams<T> l = std::move(it->second);
        layers.erase(it);
        if (!l.w) fail(ErrorKind::MissingWeights, "Layer " + std::to_string(idx) + " is missing its weights.");
        if (!l.b) fail(ErrorKind::MissingBiases, "Layer " + std::to_string(idx) + " is missing its biases.");
        const size_t wr = l.w->rows, wc = l.w->cols, br = l.b->rows, bc = l.b->cols;
        // tensors are created in the reference's order (save.rs:541-566), which fixes their ids
        ParamState<T> lin;
        lin.w = Tensor2D<T>::from_cpu_vector(ctx, l.w->v, {wr, wc});
        lin.b = Tensor2D<T>::from_cpu_vector(ctx, l.b->v, {br, bc});
        lin.master_w = from_f32(l.master_w, wr, wc);
        lin.master_b = from_f32(l.master_b, br, bc);
        lin.dv_w = from_f32(l.dv_w, wr, wc);
        lin.dv_b = from_f32(l.dv_b, br, bc);
        lin.dm_w = from_f32(l.dm_w, wr, wc);
        lin.dm_b = from_f32(l.dm_b, br, bc);
        ParamState<T> nrm;
        nrm.w = from_t(l.norm_w, br, wc);
        nrm.b = from_t(l.norm_b, br, bc);
        nrm.master_w = from_f32(l.master_norm_w, br, wc);
        nrm.master_b = from_f32(l.master_norm_b, br, bc);
        nrm.dv_w = from_f32(l.dv_norm_w, br, wc);
        nrm.dv_b = from_f32(l.dv_norm_b, br, bc);
        nrm.dm_w = from_f32(l.dm_norm_w, br, wc);
        nrm.dm_b = from_f32(l.dm_norm_b, br, bc);
        blocks.push_back(DenseBlock<T>::from_tensors(ctx, is_training, std::move(lin), std::move(nrm), max_batch_size,
                                                     LayerInitConfig{}));
    }
    return blocks;
}

template SafetensorFile SafetensorFile::from_ffn<float>(const GpuContext &, const FeedForwardNetwork<float> &);
template SafetensorFile SafetensorFile::from_ffn<f16>(const GpuContext &, const FeedForwardNetwork<f16> &);
template SafetensorFile SafetensorFile::from_blocks<float>(const GpuContext &, const std::vector<DenseBlock<float>> &);
template SafetensorFile SafetensorFile::from_blocks<f16>(const GpuContext &, const std::vector<DenseBlock<f16>> &);
template void SafetensorFile::pass_blocks<float>(const GpuContext &, const std::vector<DenseBlock<float>> &);
template void SafetensorFile::pass_blocks<f16>(const GpuContext &, const std::vector<DenseBlock<f16>> &);
template void SafetensorFile::pass_layer<float>(const GpuContext &, const DenseBlock<float> &, size_t);
template void SafetensorFile::pass_layer<f16>(const GpuContext &, const DenseBlock<f16> &, size_t);
template std::vector<DenseBlock<float>> SafetensorFile::into_blocks<float>(const GpuContext &, bool, size_t) &&;
template std::vector<DenseBlock<f16>> SafetensorFile::into_blocks<f16>(const GpuContext &, bool, size_t) &&;

}  // namespace soklyn
