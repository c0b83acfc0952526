// Safetensors weights into device-resident buffers.  The reference reads a
// file's 8-byte little-endian header length, the JSON header (one entry per
// tensor: dtype, shape, data_offsets relative to the data section, plus an
// optional "__metadata__"), and the raw bytes of one tensor
// (nemotron-model/src/weights.rs:161-267, 276-358).  Here the bytes go
// straight to the device, and an int8 per-row linear layer (I8 codes [n][k],
// F32 scales [n]) lands in the tiled weight layout the kernels read.
#include <hip/hip_runtime_api.h>

#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "nh_runtime.h"

using namespace nh;

namespace {

// ---- a small JSON reader for safetensors headers -------------------------
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    bool is_uint = false;  // an unsigned integer literal (no sign, fraction or exponent)
    uint64_t u = 0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;  // in file order

    const Json* get(const char* key) const {
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonParser {
   public:
    JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}

    bool parse(Json* out) {
        skip();
        if (!value(out, 0)) return false;
        skip();
        return p_ == end_;
    }

   private:
    const char* p_;
    const char* end_;

    void skip() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = std::strlen(w);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string* s, uint32_t c) {
        if (c < 0x80) {
            s->push_back((char)c);
        } else if (c < 0x800) {
            s->push_back((char)(0xC0 | (c >> 6)));
            s->push_back((char)(0x80 | (c & 0x3F)));
        } else if (c < 0x10000) {
            s->push_back((char)(0xE0 | (c >> 12)));
            s->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (c & 0x3F)));
        } else {
            s->push_back((char)(0xF0 | (c >> 18)));
            s->push_back((char)(0x80 | ((c >> 12) & 0x3F)));
            s->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
            s->push_back((char)(0x80 | (c & 0x3F)));
        }
    }
    bool hex4(uint32_t* v) {
        if (end_ - p_ < 4) return false;
        *v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string* s) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            const unsigned char c = (unsigned char)*p_++;
            if (c < 0x20) return false;
            if (c != '\\') {
                s->push_back((char)c);
                continue;
            }
            if (p_ >= end_) return false;
            const char e = *p_++;
            switch (e) {
                case '"': s->push_back('"'); break;
                case '\\': s->push_back('\\'); break;
                case '/': s->push_back('/'); break;
                case 'b': s->push_back('\b'); break;
                case 'f': s->push_back('\f'); break;
                case 'n': s->push_back('\n'); break;
                case 'r': s->push_back('\r'); break;
                case 't': s->push_back('\t'); break;
                case 'u': {
                    uint32_t c1;
                    if (!hex4(&c1)) return false;
                    if (c1 >= 0xD800 && c1 < 0xDC00) {  // a surrogate pair
                        uint32_t c2;
                        if (!lit("\\u") || !hex4(&c2) || c2 < 0xDC00 || c2 >= 0xE000) return false;
                        c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                    }
                    put_utf8(s, c1);
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool number(Json* v) {
        const char* start = p_;
        bool plain = true;
        if (p_ < end_ && *p_ == '-') { ++p_; plain = false; }
        if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
        if (*p_ == '0') ++p_;
        else while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        if (p_ < end_ && *p_ == '.') {
            plain = false;
            ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            plain = false;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v->kind = Json::NUM;
        if (plain) {  // as_u64: an unsigned integer that fits 64 bits
            uint64_t u = 0;
            bool fits = true;
            for (const char* q = start; q < p_; ++q) {
                const uint64_t d = (uint64_t)(*q - '0');
                if (u > (UINT64_MAX - d) / 10) fits = false;
                u = u * 10 + d;
            }
            v->is_uint = fits;
            v->u = u;
        }
        return true;
    }
    bool value(Json* v, int depth) {
        if (depth > 64 || p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v->kind = Json::OBJ;
            skip();
            if (p_ < end_ && *p_ == '}') { ++p_; return true; }
            for (;;) {
                skip();
                std::string key;
                if (!string(&key)) return false;
                skip();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                skip();
                Json item;
                if (!value(&item, depth + 1)) return false;
                v->obj.emplace_back(std::move(key), std::move(item));
                skip();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; return true; }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v->kind = Json::ARR;
            skip();
            if (p_ < end_ && *p_ == ']') { ++p_; return true; }
            for (;;) {
                skip();
                Json item;
                if (!value(&item, depth + 1)) return false;
                v->arr.push_back(std::move(item));
                skip();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; return true; }
                return false;
            }
        }
        if (c == '"') {
            v->kind = Json::STR;
            return string(&v->s);
        }
        if (lit("true")) { v->kind = Json::BOOL; v->b = true; return true; }
        if (lit("false")) { v->kind = Json::BOOL; return true; }
        if (lit("null")) { v->kind = Json::NUL; return true; }
        return number(v);
    }
};

struct FileCloser {
    void operator()(FILE* f) const {
        if (f) std::fclose(f);
    }
};
using File = std::unique_ptr<FILE, FileCloser>;

nh_status io_error(nh_error* err, const char* path, const char* what) {
    return set_error(err, NH_IO_ERROR, "%s: %s (%s)", path, what, std::strerror(errno));
}

// The header of `path` (read_header_length + read_safetensors_header,
// weights.rs:210-267) and the entry `name`, validated as
// RawTensorHeader::from_value does (weights.rs:276-358).
nh_status tensor_entry(const char* path, const char* name, nh_tensor_info* info, nh_error* err) {
    if (!path || !name) return set_error(err, NH_INVALID_PARAMS, "path and name must not be null");
    File f(std::fopen(path, "rb"));
    if (!f) return io_error(err, path, "cannot open");
    if (std::fseek(f.get(), 0, SEEK_END) != 0) return io_error(err, path, "cannot seek");
    const long flen = std::ftell(f.get());
    if (flen < 0 || std::fseek(f.get(), 0, SEEK_SET) != 0) return io_error(err, path, "cannot size");
    const uint64_t file_len = (uint64_t)flen;
    unsigned char prefix[8];
    if (std::fread(prefix, 1, 8, f.get()) != 8) return set_error(err, NH_IO_ERROR, "%s: shorter than 8 bytes", path);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | prefix[i];
    if (hlen > file_len - 8) {  // InvalidHeaderLength (8 + header_length > file length)
        if (err) {
            err->expected = file_len;
            err->actual = hlen;
        }
        return set_error(err, NH_INVALID_HEADER, "%s: header length %llu exceeds the file (%llu bytes)", path,
                         (unsigned long long)hlen, (unsigned long long)file_len);
    }
    std::vector<char> header(hlen);
    if (hlen && std::fread(header.data(), 1, hlen, f.get()) != hlen) return io_error(err, path, "short header read");
    Json root;
    if (!JsonParser(header.data(), header.size()).parse(&root) || root.kind != Json::OBJ)
        return set_error(err, NH_INVALID_HEADER, "%s: header is not a JSON object", path);
    // every entry is validated, as reading the header does, before the lookup
    const Json* found = nullptr;
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const char* tname = kv.first.c_str();
        const Json* entry = &kv.second;
        auto bad = [&](const char* reason) {
            return set_error(err, NH_INVALID_HEADER, "invalid tensor header for %s in %s: %s", tname, path, reason);
        };
        if (entry->kind != Json::OBJ) return bad("tensor entry must be an object");
        const Json* dtype = entry->get("dtype");
        if (!dtype || dtype->kind != Json::STR) return bad("missing dtype");
        const Json* shape = entry->get("shape");
        if (!shape || shape->kind != Json::ARR) return bad("missing shape");
        for (const Json& d : shape->arr)
            if (d.kind != Json::NUM || !d.is_uint) return bad("shape entries must be unsigned integers");
        const Json* offs = entry->get("data_offsets");
        if (!offs || offs->kind != Json::ARR) return bad("missing data_offsets");
        if (offs->arr.size() != 2) return bad("data_offsets must contain [start, end]");
        if (offs->arr[0].kind != Json::NUM || !offs->arr[0].is_uint)
            return bad("data_offsets start must be an unsigned integer");
        if (offs->arr[1].kind != Json::NUM || !offs->arr[1].is_uint)
            return bad("data_offsets end must be an unsigned integer");
        if (offs->arr[1].u < offs->arr[0].u) return bad("data_offsets end must be greater than or equal to start");
        if (kv.first == name) found = entry;
    }
    if (!found) return set_error(err, NH_TENSOR_NOT_FOUND, "tensor not found: %s", name);
    auto bad = [&](const char* reason) {
        return set_error(err, NH_INVALID_HEADER, "invalid tensor header for %s in %s: %s", name, path, reason);
    };
    const Json* dtype = found->get("dtype");
    const Json* shape = found->get("shape");
    const Json* offs = found->get("data_offsets");
    const uint64_t start = offs->arr[0].u, end = offs->arr[1].u;
    if (dtype->s.size() >= sizeof(info->dtype)) return bad("dtype longer than 15 characters");
    if (shape->arr.size() > 8) return bad("more than 8 dimensions");
    std::memset(info, 0, sizeof(*info));
    std::memcpy(info->dtype, dtype->s.data(), dtype->s.size());
    info->ndim = (uint32_t)shape->arr.size();
    for (size_t i = 0; i < shape->arr.size(); ++i) info->shape[i] = shape->arr[i].u;
    info->data_begin = 8 + hlen + start;
    info->data_bytes = end - start;
    return NH_OK;
}

// The tensor's bytes from the file (load_tensor, weights.rs:167-204).
nh_status read_bytes(const char* path, const nh_tensor_info& info, std::vector<unsigned char>* out, nh_error* err) {
    File f(std::fopen(path, "rb"));
    if (!f) return io_error(err, path, "cannot open");
    out->resize(info.data_bytes);
    if (std::fseek(f.get(), (long)info.data_begin, SEEK_SET) != 0) return io_error(err, path, "cannot seek");
    if (info.data_bytes && std::fread(out->data(), 1, info.data_bytes, f.get()) != info.data_bytes)
        return set_error(err, NH_IO_ERROR, "%s: tensor data past the end of the file", path);
    return NH_OK;
}

}  // namespace

extern "C" {

nh_status nh_safetensors_tensor_info(const char* path, const char* name, nh_tensor_info* info, nh_error* err) {
    clear_error(err);
    if (!info) return set_error(err, NH_INVALID_PARAMS, "info must not be null");
    return tensor_entry(path, name, info, err);
}

nh_status nh_safetensors_read(nh_context* ctx, const char* path, const char* name, void* dst, size_t dst_len,
                              nh_error* err) {
    clear_error(err);
    nh_tensor_info info;
    nh_status st = tensor_entry(path, name, &info, err);
    if (st) return st;
    if (dst_len != info.data_bytes) return mismatch(err, "dst", info.data_bytes, dst_len);
    std::vector<unsigned char> bytes;
    if ((st = read_bytes(path, info, &bytes, err))) return st;
    if ((st = bind_device(ctx, err))) return st;
    if (bytes.empty()) return NH_OK;
    hipError_t e = hipMemcpy(dst, bytes.data(), bytes.size(), hipMemcpyHostToDevice);
    return e == hipSuccess ? NH_OK : device_error(err, e, "hipMemcpy(HtoD)");
}

nh_status nh_load_linear_i8(nh_context* ctx, const char* path, const char* codes_name, const char* scales_name,
                            size_t n, size_t k, void* staging, size_t staging_len, int8_t* tiled, size_t tiled_len,
                            float* scales, nh_error* err) {
    clear_error(err);
    nh_tensor_info ci, si;
    nh_status st;
    if ((st = tensor_entry(path, codes_name, &ci, err)) || (st = tensor_entry(path, scales_name, &si, err))) return st;
    size_t nk;
    if (n == 0 || k == 0 || !mul_ok(n, k, &nk)) return set_error(err, NH_INVALID_SHAPE, "invalid weight shape");
    if (std::strcmp(ci.dtype, "I8") != 0 || ci.ndim != 2 || ci.shape[0] != n || ci.shape[1] != k)
        return set_error(err, NH_INVALID_SHAPE, "%s must be I8 [%zu, %zu] (got %s with %u dims)", codes_name, n, k,
                         ci.dtype, ci.ndim);
    if (std::strcmp(si.dtype, "F32") != 0 || si.ndim != 1 || si.shape[0] != n)
        return set_error(err, NH_INVALID_SHAPE, "%s must be F32 [%zu] (got %s with %u dims)", scales_name, n,
                         si.dtype, si.ndim);
    if (ci.data_bytes != nk) return mismatch(err, "codes", nk, ci.data_bytes);
    if (si.data_bytes != n * sizeof(float)) return mismatch(err, "scales", n * sizeof(float), si.data_bytes);
    if (staging_len < nk) return mismatch(err, "staging", nk, staging_len);
    const size_t need = nh_tiled_weights_bytes(n, k);
    if (tiled_len != need) return mismatch(err, "tiled", need, tiled_len);
    std::vector<unsigned char> codes, sc;
    if ((st = read_bytes(path, ci, &codes, err)) || (st = read_bytes(path, si, &sc, err))) return st;
    if ((st = bind_device(ctx, err))) return st;
    hipError_t e = hipMemcpy(staging, codes.data(), nk, hipMemcpyHostToDevice);
    if (e != hipSuccess) return device_error(err, e, "hipMemcpy(HtoD)");
    e = hipMemcpy(scales, sc.data(), sc.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) return device_error(err, e, "hipMemcpy(HtoD)");
    if ((st = nh_tile_weights_i8(ctx, (const int8_t*)staging, n, k, tiled, tiled_len, nullptr, err))) return st;
    e = hipDeviceSynchronize();
    return e == hipSuccess ? NH_OK : device_error(err, e, "hipDeviceSynchronize");
}

}  // extern "C"
