// Reader and writer of the reference's `.snl` weight file (src/weights.rs:1-121,
// src/convert.rs:316-427).  See snl_file.h for the layout.
#include "snl_file.h"

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdarg>

namespace snl {

namespace {

constexpr char kMagic[4] = {'S', 'N', 'L', 'Q'};
constexpr uint32_t kVersion = 1;
constexpr uint64_t kAlign = 256;
constexpr int kMaxDepth = 64;

uint64_t align256(uint64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool failf(std::string* err, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (err) *err = buf;
    return false;
}

// ---- a small JSON reader: objects, arrays, strings, numbers, true/false/null ----
struct JVal {
    enum Type { NUL, BOOL, NUM, STR, ARR, OBJ } type = NUL;
    bool b = false;
    std::string s;  // STR: the text; NUM: the literal
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;
    const JVal* get(const char* key) const {
        if (type != OBJ) return nullptr;
        for (const auto& kv : o)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JParser {
public:
    JParser(const char* p, size_t n) : p_(p), end_(p + n) {}
    bool parse(JVal* v, std::string* err) {
        if (!value(v, 0) || (ws(), p_ != end_)) return failf(err, "malformed JSON header near byte %zu", off());
        return true;
    }

private:
    const char* p_;
    const char* end_;
    const char* start_ = p_;
    size_t off() const { return (size_t)(p_ - start_); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(end_ - p_) < n || memcmp(p_, w, n)) return false;
        p_ += n;
        return true;
    }
    bool str(std::string* out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c != '\\') {
                out->push_back(c);
                continue;
            }
            if (p_ >= end_) return false;
            c = *p_++;
            switch (c) {
                case '"': case '\\': case '/': out->push_back(c); break;
                case 'b': out->push_back('\b'); break;
                case 'f': out->push_back('\f'); break;
                case 'n': out->push_back('\n'); break;
                case 'r': out->push_back('\r'); break;
                case 't': out->push_back('\t'); break;
                case 'u': {
                    if (end_ - p_ < 4) return false;
                    unsigned cp = 0;
                    for (int i = 0; i < 4; ++i) {
                        const char h = *p_++;
                        const int dv = h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                                     : h >= 'A' && h <= 'F' ? h - 'A' + 10 : -1;
                        if (dv < 0) return false;
                        cp = cp * 16 + (unsigned)dv;
                    }
                    if (cp < 0x80) {
                        out->push_back((char)cp);
                    } else if (cp < 0x800) {
                        out->push_back((char)(0xC0 | (cp >> 6)));
                        out->push_back((char)(0x80 | (cp & 0x3F)));
                    } else {
                        out->push_back((char)(0xE0 | (cp >> 12)));
                        out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                        out->push_back((char)(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool value(JVal* v, int depth) {
        if (depth > kMaxDepth) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v->type = JVal::OBJ;
            ws();
            if (p_ < end_ && *p_ == '}') return ++p_, true;
            for (;;) {
                ws();
                std::string k;
                if (!str(&k)) return false;
                ws();
                if (p_ >= end_ || *p_++ != ':') return false;
                v->o.emplace_back(std::move(k), JVal{});
                if (!value(&v->o.back().second, depth + 1)) return false;
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') return ++p_, true;
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v->type = JVal::ARR;
            ws();
            if (p_ < end_ && *p_ == ']') return ++p_, true;
            for (;;) {
                v->a.emplace_back();
                if (!value(&v->a.back(), depth + 1)) return false;
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') return ++p_, true;
                return false;
            }
        }
        if (c == '"') {
            v->type = JVal::STR;
            return str(&v->s);
        }
        if (lit("true")) return v->type = JVal::BOOL, v->b = true, true;
        if (lit("false")) return v->type = JVal::BOOL, v->b = false, true;
        if (lit("null")) return v->type = JVal::NUL, true;
        const char* q = p_;
        // (strchr also finds the terminator: a NUL byte is no part of a number)
        while (q < end_ && *q != '\0' && strchr("+-0123456789.eE", *q) != nullptr) ++q;
        if (q == p_) return false;
        v->type = JVal::NUM;
        v->s.assign(p_, q);
        p_ = q;
        return true;
    }
};

bool get_u64(const JVal* v, uint64_t* out) {
    if (!v || v->type != JVal::NUM || v->s.empty() || v->s[0] == '-' || v->s.find_first_of(".eE") != std::string::npos)
        return false;
    errno = 0;
    char* e = nullptr;
    const unsigned long long x = strtoull(v->s.c_str(), &e, 10);
    if (errno || *e) return false;
    *out = x;
    return true;
}

bool get_int(const JVal& obj, const char* key, int64_t lo, int64_t hi, int32_t* out, std::string* err) {
    uint64_t x;
    if (!get_u64(obj.get(key), &x) || (int64_t)x < lo || (int64_t)x > hi)
        return failf(err, "header config: `%s` missing or out of range", key);
    *out = (int32_t)x;
    return true;
}

bool get_f32(const JVal& obj, const char* key, float* out, std::string* err) {
    const JVal* v = obj.get(key);
    if (!v || v->type != JVal::NUM) return failf(err, "header config: `%s` missing", key);
    char* e = nullptr;
    *out = strtof(v->s.c_str(), &e);
    if (*e || !std::isfinite(*out)) return failf(err, "header config: `%s` is not a finite number", key);
    return true;
}

const char* dtype_name(int d) { return d == FD_Q8_0 ? "q8_0" : d == FD_Q4_0 ? "q4_0" : "f32"; }

// shortest decimal that reads back as the same f32 (the reference's serde_json prints f32 so)
std::string f32_text(float x) {
    char buf[48];
    for (int p = 1; p <= 9; ++p) {
        snprintf(buf, sizeof buf, "%.*g", p, (double)x);
        if (strtof(buf, nullptr) == x) break;
    }
    std::string s = buf;
    if (s.find_first_of(".eEn") == std::string::npos) s += ".0";  // a float literal, as serde writes it
    return s;
}

void json_str(std::string* o, const std::string& s) {
    o->push_back('"');
    for (const unsigned char c : s) {
        if (c == '"' || c == '\\') {
            o->push_back('\\');
            o->push_back((char)c);
        } else if (c < 0x20) {
            char b[8];
            snprintf(b, sizeof b, "\\u%04x", c);
            *o += b;
        } else {
            o->push_back((char)c);
        }
    }
    o->push_back('"');
}

// ModelConfig (src/config.rs:6-37) in declaration order
std::string config_json(const FileConfig& f) {
    const snl_config& c = f.cfg;
    std::string o = "{";
    auto num = [&](const char* k, long long v) {
        json_str(&o, k);
        o += ":" + std::to_string(v) + ",";
    };
    num("hidden", c.hidden);
    num("intermediate", c.intermediate);
    num("vocab", c.vocab);
    num("n_layers", c.n_layers);
    o += "\"full_attention\":[";
    for (int i = 0; i < c.n_layers; ++i) o += std::string(i ? "," : "") + (c.full_attention[i] ? "true" : "false");
    o += "],";
    num("n_heads", c.n_heads);
    num("n_kv_heads", c.n_kv_heads);
    num("head_dim", c.head_dim);
    num("rot_dim", c.rot_dim);
    o += "\"rope_theta\":" + f32_text(c.rope_theta) + ",";
    o += "\"mrope_section\":[" + std::to_string(c.mrope_section[0]) + "," + std::to_string(c.mrope_section[1]) + "," +
         std::to_string(c.mrope_section[2]) + "],";
    num("lin_k_heads", c.lin_k_heads);
    num("lin_v_heads", c.lin_v_heads);
    num("lin_k_dim", c.lin_k_dim);
    num("lin_v_dim", c.lin_v_dim);
    num("conv_kernel", c.conv_kernel);
    o += "\"eps\":" + f32_text(c.eps) + ",";
    num("loop_start", c.loop_start);
    num("loop_end", c.loop_end);
    num("loop_count", c.loop_count);
    if (c.mhc_streams > 0)
        o += "\"mhc\":{\"start\":" + std::to_string(c.mhc_start) + ",\"end\":" + std::to_string(c.mhc_end) +
             ",\"streams\":" + std::to_string(c.mhc_streams) + ",\"iterations\":" + std::to_string(c.mhc_iterations) +
             "},";
    else
        o += "\"mhc\":null,";
    o += "\"eos\":[";
    for (int i = 0; i < c.n_eos; ++i) o += std::string(i ? "," : "") + std::to_string(c.eos[i]);
    o += "],";
    num("max_position", f.max_position);
    o += "\"vision\":null}";
    return o;
}

std::string header_json(const std::string& model_name, const std::string& quant, const FileConfig& cfg,
                        const std::map<std::string, FileTensor>& tensors) {
    std::string o = "{\"model_name\":";
    json_str(&o, model_name);
    o += ",\"quant\":";
    json_str(&o, quant);
    o += ",\"config\":" + config_json(cfg) + ",\"tensors\":{";
    bool first = true;
    for (const auto& kv : tensors) {  // sorted by name, as the reference's BTreeMap
        if (!first) o += ",";
        first = false;
        json_str(&o, kv.first);
        o += ":{\"dtype\":\"" + std::string(dtype_name(kv.second.dtype)) + "\",\"shape\":[";
        for (size_t i = 0; i < kv.second.shape.size(); ++i)
            o += std::string(i ? "," : "") + std::to_string(kv.second.shape[i]);
        o += "],\"offset\":" + std::to_string(kv.second.offset) +
             ",\"scales_offset\":" + std::to_string(kv.second.scales_offset) + "}";
    }
    o += "}}";
    return o;
}

}  // namespace

uint64_t FileTensor::quant_bytes() const {
    const uint64_t n = (uint64_t)(rows() * cols());
    return dtype == FD_F32 ? n * 4 : dtype == FD_Q8_0 ? n : n / 2;
}

uint64_t FileTensor::scale_bytes() const {
    const uint64_t n = (uint64_t)(rows() * cols());
    return dtype == FD_F32 ? 0 : n / 32 * 4;
}

SnlFile::~SnlFile() {
    if (base_) munmap(base_, size_);
}

// WeightFile::open (src/weights.rs:86-105) and the tensor table
bool SnlFile::open(const char* path, std::string* err) {
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return failf(err, "opening %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return failf(err, "opening %s: %s", path, strerror(errno));
    }
    size_ = (size_t)st.st_size;
    void* m = size_ ? mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
    ::close(fd);
    if (m == MAP_FAILED) return failf(err, "%s is not a SenseNova Loop weight file", path);
    base_ = static_cast<uint8_t*>(m);
    if (size_ < 16 || memcmp(base_, kMagic, 4) != 0) return failf(err, "%s is not a SenseNova Loop weight file", path);
    uint32_t version;
    uint64_t len;
    memcpy(&version, base_ + 4, 4);
    memcpy(&len, base_ + 8, 8);
    if (version != kVersion) return failf(err, "unsupported weight file version %u", version);
    if (len > size_ - 16) return failf(err, "%s: header runs past the end of the file", path);
    JVal h;
    if (!JParser(reinterpret_cast<const char*>(base_) + 16, (size_t)len).parse(&h, err)) return false;
    const JVal *mn = h.get("model_name"), *q = h.get("quant"), *cf = h.get("config"), *ts = h.get("tensors");
    if (!mn || mn->type != JVal::STR || !q || q->type != JVal::STR || !cf || cf->type != JVal::OBJ || !ts ||
        ts->type != JVal::OBJ)
        return failf(err, "%s: header lacks model_name, quant, config or tensors", path);
    model_name_ = mn->s;
    quant_ = q->s;
    header_json_.assign(reinterpret_cast<const char*>(base_) + 16, (size_t)len);
    for (const auto& kv : ts->o) {
        const JVal& t = kv.second;
        FileTensor ft;
        const JVal* d = t.get("dtype");
        const JVal* sh = t.get("shape");
        if (!d || d->type != JVal::STR || !sh || sh->type != JVal::ARR || sh->a.empty() || sh->a.size() > 2 ||
            !get_u64(t.get("offset"), &ft.offset) || !get_u64(t.get("scales_offset"), &ft.scales_offset))
            return failf(err, "%s: malformed entry for tensor `%s`", path, kv.first.c_str());
        if (d->s == "f32") ft.dtype = FD_F32;
        else if (d->s == "q8_0") ft.dtype = FD_Q8_0;
        else if (d->s == "q4_0") ft.dtype = FD_Q4_0;
        else return failf(err, "%s: tensor `%s` has unknown dtype `%s`", path, kv.first.c_str(), d->s.c_str());
        for (const JVal& e : sh->a) {
            uint64_t x;
            // (dims up to 2^30 keep rows * cols * 4 inside 64 bits for the bounds checks below)
            if (!get_u64(&e, &x) || x == 0 || x > (1ull << 30)) return failf(err, "%s: bad shape of `%s`", path, kv.first.c_str());
            ft.shape.push_back((int64_t)x);
        }
        if (ft.dtype != FD_F32 && ft.cols() % 32)
            return failf(err, "%s: `%s`: columns not divisible by 32", path, kv.first.c_str());
        if (ft.offset > size_ || ft.quant_bytes() > size_ - ft.offset || ft.scales_offset > size_ ||
            ft.scale_bytes() > size_ - ft.scales_offset)
            return failf(err, "%s: tensor `%s` runs past the end of the file", path, kv.first.c_str());
        tensors_[kv.first] = ft;
    }
    return true;
}

const FileTensor* SnlFile::find(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
}

// ModelConfig from the header (src/config.rs:6-37); vision is ignored
bool SnlFile::config(FileConfig* out, std::string* err) const {
    JVal h;
    if (!JParser(header_json_.data(), header_json_.size()).parse(&h, err)) return false;
    const JVal* cp = h.get("config");
    if (!cp || cp->type != JVal::OBJ) return failf(err, "header lacks config");
    const JVal& c = *cp;
    snl_config k{};
    const int64_t big = 1 << 30;
    if (!get_int(c, "hidden", 1, big, &k.hidden, err) || !get_int(c, "intermediate", 1, big, &k.intermediate, err) ||
        !get_int(c, "vocab", 1, big, &k.vocab, err) || !get_int(c, "n_layers", 1, 64, &k.n_layers, err) ||
        !get_int(c, "n_heads", 1, big, &k.n_heads, err) || !get_int(c, "n_kv_heads", 1, big, &k.n_kv_heads, err) ||
        !get_int(c, "head_dim", 1, big, &k.head_dim, err) || !get_int(c, "rot_dim", 0, big, &k.rot_dim, err) ||
        !get_f32(c, "rope_theta", &k.rope_theta, err) || !get_int(c, "lin_k_heads", 0, big, &k.lin_k_heads, err) ||
        !get_int(c, "lin_v_heads", 0, big, &k.lin_v_heads, err) || !get_int(c, "lin_k_dim", 0, big, &k.lin_k_dim, err) ||
        !get_int(c, "lin_v_dim", 0, big, &k.lin_v_dim, err) || !get_int(c, "conv_kernel", 0, big, &k.conv_kernel, err) ||
        !get_f32(c, "eps", &k.eps, err) || !get_int(c, "loop_start", 0, 64, &k.loop_start, err) ||
        !get_int(c, "loop_end", 0, 64, &k.loop_end, err) || !get_int(c, "loop_count", 0, 64, &k.loop_count, err))
        return false;
    const JVal* fa = c.get("full_attention");
    if (!fa || fa->type != JVal::ARR || (int)fa->a.size() != k.n_layers)
        return failf(err, "header config: `full_attention` must list n_layers flags");
    for (int i = 0; i < k.n_layers; ++i) {
        if (fa->a[i].type != JVal::BOOL) return failf(err, "header config: `full_attention` must be booleans");
        k.full_attention[i] = fa->a[i].b ? 1 : 0;
    }
    const JVal* mr = c.get("mrope_section");
    if (mr && mr->type != JVal::NUL) {
        if (mr->type != JVal::ARR || mr->a.size() != 3) return failf(err, "header config: bad `mrope_section`");
        for (int i = 0; i < 3; ++i) {
            uint64_t x;
            if (!get_u64(&mr->a[i], &x) || x > 1024) return failf(err, "header config: bad `mrope_section`");
            k.mrope_section[i] = (int32_t)x;
        }
    } else {  // default_mrope (src/config.rs:72-74)
        k.mrope_section[0] = 11, k.mrope_section[1] = 11, k.mrope_section[2] = 10;
    }
    const JVal* mh = c.get("mhc");
    if (mh && mh->type == JVal::OBJ) {
        if (!get_int(*mh, "start", 0, 64, &k.mhc_start, err) || !get_int(*mh, "end", 0, 64, &k.mhc_end, err) ||
            !get_int(*mh, "streams", 1, 64, &k.mhc_streams, err) ||
            !get_int(*mh, "iterations", 0, 1 << 16, &k.mhc_iterations, err))
            return false;
    } else if (mh && mh->type != JVal::NUL) {
        return failf(err, "header config: bad `mhc`");
    }
    const JVal* eos = c.get("eos");
    if (!eos || eos->type != JVal::ARR || eos->a.size() > 4) return failf(err, "header config: `eos` must list at most 4 ids");
    k.n_eos = (int32_t)eos->a.size();
    for (int i = 0; i < k.n_eos; ++i) {
        uint64_t x;
        if (!get_u64(&eos->a[i], &x) || x > 0xFFFFFFFFull) return failf(err, "header config: bad `eos`");
        k.eos[i] = (uint32_t)x;
    }
    uint64_t mp = 0;
    if (!get_u64(c.get("max_position"), &mp) || mp == 0) return failf(err, "header config: `max_position` missing");
    out->cfg = k;
    out->max_position = (int64_t)mp;
    return true;
}

SnlWriter::~SnlWriter() {
    if (fd_ >= 0) {
        ::close(fd_);
        unlink(tmp_.c_str());
    }
}

// convert() (src/convert.rs:330-360): regions laid out in order, each quant and scale region
// 256-aligned, data from align(16 + header + 4096)
bool SnlWriter::begin(const char* path, const std::string& model_name, const std::string& quant, const FileConfig& cfg,
                      const std::vector<WriteTensor>& tensors, std::vector<FileTensor>* placed, std::string* err) {
    std::map<std::string, FileTensor> table;
    placed->clear();
    uint64_t cursor = 0;
    for (const WriteTensor& t : tensors) {
        FileTensor ft;
        ft.dtype = t.dtype;
        ft.shape = t.shape;
        if (ft.dtype != FD_F32 && ft.cols() % 32) return failf(err, "%s: columns not divisible by 32", t.name.c_str());
        ft.offset = cursor;
        cursor = align256(cursor + ft.quant_bytes());
        ft.scales_offset = cursor;
        cursor = align256(cursor + ft.scale_bytes());
        if (table.count(t.name)) return failf(err, "duplicate tensor `%s`", t.name.c_str());
        table[t.name] = ft;
    }
    const std::string probe = header_json(model_name, quant, cfg, table);
    const uint64_t data_start = align256(16 + probe.size() + 4096);
    for (auto& kv : table) {
        kv.second.offset += data_start;
        kv.second.scales_offset += data_start;
    }
    for (const WriteTensor& t : tensors) placed->push_back(table[t.name]);
    const std::string hdr = header_json(model_name, quant, cfg, table);
    if (16 + hdr.size() > data_start) return failf(err, "internal error: header larger than reserved space");
    path_ = path;
    tmp_ = path_ + ".partial";
    fd_ = ::open(tmp_.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (fd_ < 0) return failf(err, "creating %s: %s", tmp_.c_str(), strerror(errno));
    uint8_t pre[16];
    memcpy(pre, kMagic, 4);
    memcpy(pre + 4, &kVersion, 4);
    const uint64_t len = hdr.size();
    memcpy(pre + 8, &len, 8);
    if (!write_region(0, pre, 16, err) || !write_region(16, hdr.data(), hdr.size(), err)) return false;
    // the file covers the final alignment padding (src/convert.rs:417-422)
    if (ftruncate(fd_, (off_t)(data_start + cursor)) != 0) return failf(err, "sizing %s: %s", tmp_.c_str(), strerror(errno));
    return true;
}

bool SnlWriter::write_region(uint64_t offset, const void* data, size_t bytes, std::string* err) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    while (bytes) {
        const ssize_t n = pwrite(fd_, p, bytes, (off_t)offset);
        if (n < 0) {
            if (errno == EINTR) continue;
            return failf(err, "writing %s: %s", tmp_.c_str(), strerror(errno));
        }
        p += n;
        offset += (uint64_t)n;
        bytes -= (size_t)n;
    }
    return true;
}

bool SnlWriter::finish(std::string* err) {
    if (fsync(fd_) != 0 || ::close(fd_) != 0) {
        fd_ = -1;
        return failf(err, "closing %s: %s", tmp_.c_str(), strerror(errno));
    }
    fd_ = -1;
    if (rename(tmp_.c_str(), path_.c_str()) != 0) return failf(err, "renaming %s: %s", tmp_.c_str(), strerror(errno));
    return true;
}

}  // namespace snl
