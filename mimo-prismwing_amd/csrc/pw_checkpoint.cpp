// Checkpoint-bound weights -> HBM-resident expert bank.
//
// The reference maps safetensors files read-only and binds page-rounded no-copy regions per call
// (MappedSafetensors::open / tensor / tensor_no_copy_region, src/lib.rs:783-972; expert tensors
// model.layers.{L}.mlp.experts.{E}.{gate,up,down}_proj.weight and ..._scale_inv,
// src/text_endpoint.rs:4785-4845). Here the header is parsed the same way (length prefix, JSON
// object of {dtype, shape, data_offsets}, optional __metadata__, checked sizes, no overlaps, no
// duplicate names) and a layer's experts are validated like validate_fp8_views_internal
// (src/lib.rs:1217-1270) and copied once into one device allocation that the bank owns.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/pwfp8.h"
#include "pw_device.h"
#include "pw_internal.h"

namespace {

constexpr uint64_t kMaxHeaderBytes = 256ull * 1024 * 1024;  // MAX_HEADER_BYTES, src/lib.rs:77

// ---- a small JSON reader for safetensors headers (objects, arrays, strings, integers, literals)
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    bool integral = false;  // a non-negative integer that fits uint64
    uint64_t u = 0;
    std::string s;
    std::vector<Json> a;
    std::vector<std::pair<std::string, Json>> o;
};

struct JsonReader {
    const char *p, *end;
    std::string err;

    void ws()
    {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r'))
            ++p;
    }
    bool fail(const char *m)
    {
        if (err.empty())
            err = m;
        return false;
    }
    bool hex4(uint32_t &v)
    {
        if (end - p < 4)
            return fail("truncated \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("bad \\u escape");
        }
        return true;
    }
    static void utf8(std::string &out, uint32_t cp)
    {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool str(std::string &out)
    {
        if (p >= end || *p != '"')
            return fail("expected a string");
        ++p;
        while (p < end && *p != '"') {
            const unsigned char c = (unsigned char)*p++;
            if (c < 0x20)
                return fail("control character in string");
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (p >= end)
                return fail("truncated escape");
            const char e = *p++;
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
                uint32_t cp;
                if (!hex4(cp))
                    return false;
                if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                    uint32_t lo;
                    if (end - p < 2 || p[0] != '\\' || p[1] != 'u')
                        return fail("unpaired surrogate");
                    p += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo > 0xDFFF)
                        return fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(out, cp);
                break;
            }
            default: return fail("bad escape");
            }
        }
        if (p >= end)
            return fail("unterminated string");
        ++p;
        return true;
    }
    bool num(Json &v)
    {
        const char *s0 = p;
        if (p < end && *p == '-')
            ++p;
        bool digits = false, frac = false;
        uint64_t u = 0;
        bool overflow = false;
        while (p < end && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p - '0');
            if (u > (UINT64_MAX - d) / 10)
                overflow = true;
            u = u * 10 + d;
            ++p;
            digits = true;
        }
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {
            frac = true;
            ++p;
            while (p < end && ((*p >= '0' && *p <= '9') || *p == '+' || *p == '-' || *p == 'e' || *p == 'E'))
                ++p;
        }
        if (!digits)
            return fail("bad number");
        v.kind = Json::NUM;
        v.integral = *s0 != '-' && !frac && !overflow;
        v.u = u;
        return true;
    }
    bool value(Json &v, int depth)
    {
        if (depth > 64)
            return fail("nesting too deep");
        ws();
        if (p >= end)
            return fail("unexpected end");
        const char c = *p;
        if (c == '{') {
            ++p;
            v.kind = Json::OBJ;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!str(key))
                    return false;
                for (const auto &kv : v.o)
                    if (kv.first == key)
                        return fail("duplicate object key");
                ws();
                if (p >= end || *p != ':')
                    return fail("expected ':'");
                ++p;
                Json child;
                if (!value(child, depth + 1))
                    return false;
                v.o.emplace_back(std::move(key), std::move(child));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            ++p;
            v.kind = Json::ARR;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            for (;;) {
                Json child;
                if (!value(child, depth + 1))
                    return false;
                v.a.push_back(std::move(child));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::STR;
            return str(v.s);
        }
        if (end - p >= 4 && !memcmp(p, "true", 4)) {
            p += 4;
            v.kind = Json::BOOL;
            v.b = true;
            return true;
        }
        if (end - p >= 5 && !memcmp(p, "false", 5)) {
            p += 5;
            v.kind = Json::BOOL;
            return true;
        }
        if (end - p >= 4 && !memcmp(p, "null", 4)) {
            p += 4;
            v.kind = Json::NUL;
            return true;
        }
        return num(v);
    }
};

// dtype_bytes (src/lib.rs:750-758)
int dtype_bytes(const std::string &d)
{
    if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "F8_E4M3FN" || d == "F8_E5M2")
        return 1;
    if (d == "U16" || d == "I16" || d == "F16" || d == "BF16")
        return 2;
    if (d == "U32" || d == "I32" || d == "F32")
        return 4;
    if (d == "U64" || d == "I64" || d == "F64")
        return 8;
    return 0;
}

struct TensorRecord {
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t start = 0, end = 0;
};

}  // namespace

struct pw_safetensors {
    int fd = -1;
    uint8_t *map = nullptr;
    size_t size = 0;
    size_t payload_start = 0;
    std::string path;
    std::map<std::string, TensorRecord> tensors;
};

extern "C" {

int pw_safetensors_open(const char *path, pw_safetensors **out)
{
    if (!path || !out)
        return pw::fail(PW_ERR_ARGUMENT, "null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0)
        return pw::fail(PW_ERR_ARGUMENT, "%s: cannot open", path);
    struct stat stt;
    if (fstat(fd, &stt) != 0 || stt.st_size < 16) {
        close(fd);
        return pw::fail(PW_ERR_LAYOUT, "safetensors file is too short");
    }
    const size_t size = (size_t)stt.st_size;
    void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
        close(fd);
        return pw::fail(PW_ERR_DEVICE, "%s: mmap failed", path);
    }
    pw_safetensors *st = new pw_safetensors;
    st->fd = fd;
    st->map = (uint8_t *)m;
    st->size = size;
    st->path = path;
    auto bad = [&](const char *fmt, ...) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        pw_safetensors_close(st);
        return pw::fail(PW_ERR_LAYOUT, "%s", buf);
    };
    uint64_t header_bytes = 0;
    for (int i = 7; i >= 0; --i)
        header_bytes = (header_bytes << 8) | st->map[i];
    if (header_bytes == 0 || header_bytes > kMaxHeaderBytes || header_bytes % 8 != 0 ||
        8 + header_bytes > (uint64_t)size)
        return bad("invalid safetensors header length %llu", (unsigned long long)header_bytes);
    st->payload_start = 8 + (size_t)header_bytes;
    JsonReader r{(const char *)st->map + 8, (const char *)st->map + st->payload_start, {}};
    Json root;
    if (!r.value(root, 0))
        return bad("malformed safetensors header: %s", r.err.c_str());
    r.ws();
    if (r.p != r.end)
        return bad("trailing header data");
    if (root.kind != Json::OBJ)
        return bad("safetensors header must be an object");
    const uint64_t payload_bytes = (uint64_t)size - st->payload_start;
    std::vector<std::pair<std::pair<uint64_t, uint64_t>, std::string>> ranges;
    for (const auto &kv : root.o) {
        const std::string &name = kv.first;
        const Json &v = kv.second;
        if (name == "__metadata__") {
            if (v.kind != Json::OBJ)
                return bad("__metadata__ must be an object");
            continue;
        }
        if (v.kind != Json::OBJ)
            return bad("%s: expected an object", name.c_str());
        const Json *dtype = nullptr, *shape = nullptr, *offsets = nullptr;
        for (const auto &f : v.o) {
            if (f.first == "dtype") dtype = &f.second;
            else if (f.first == "shape") shape = &f.second;
            else if (f.first == "data_offsets") offsets = &f.second;
        }
        if (!dtype || dtype->kind != Json::STR)
            return bad("%s: missing dtype", name.c_str());
        const int eb = dtype_bytes(dtype->s);
        if (!eb)
            return bad("%s: unknown dtype %s", name.c_str(), dtype->s.c_str());
        if (!shape || shape->kind != Json::ARR)
            return bad("%s: missing shape", name.c_str());
        TensorRecord rec;
        rec.dtype = dtype->s;
        uint64_t elements = 1;
        for (const Json &d : shape->a) {
            if (d.kind != Json::NUM || !d.integral)
                return bad("%s: invalid shape", name.c_str());
            if (d.u == 0)
                return bad("%s: empty or zero tensor shape", name.c_str());
            if (elements > UINT64_MAX / d.u)
                return bad("%s: shape overflow", name.c_str());
            elements *= d.u;
            rec.shape.push_back(d.u);
        }
        if (rec.shape.empty())
            return bad("%s: empty or zero tensor shape", name.c_str());
        if (!offsets || offsets->kind != Json::ARR || offsets->a.size() != 2 || offsets->a[0].kind != Json::NUM ||
            !offsets->a[0].integral || offsets->a[1].kind != Json::NUM || !offsets->a[1].integral)
            return bad("%s: missing offsets", name.c_str());
        rec.start = offsets->a[0].u;
        rec.end = offsets->a[1].u;
        if (rec.end < rec.start)
            return bad("tensor offsets reversed");
        if (elements > UINT64_MAX / (uint64_t)eb)
            return bad("%s: tensor byte overflow", name.c_str());
        if (rec.end - rec.start != elements * (uint64_t)eb)
            return bad("%s: shape/dtype requires %llu bytes, got %llu", name.c_str(),
                       (unsigned long long)(elements * eb), (unsigned long long)(rec.end - rec.start));
        if (rec.end > payload_bytes)
            return bad("%s: tensor payload exceeds file", name.c_str());
        ranges.push_back({{rec.start, rec.end}, name});
        st->tensors.emplace(name, std::move(rec));
    }
    if (st->tensors.empty())
        return bad("safetensors file contains no tensors");
    std::sort(ranges.begin(), ranges.end());
    uint64_t prev_end = 0;
    for (const auto &rg : ranges) {
        if (rg.first.first < prev_end)
            return bad("%s: overlapping tensor payload", rg.second.c_str());
        prev_end = rg.first.second;
    }
    *out = st;
    return PW_OK;
}

void pw_safetensors_close(pw_safetensors *st)
{
    if (!st)
        return;
    if (st->map)
        munmap(st->map, st->size);
    if (st->fd >= 0)
        close(st->fd);
    delete st;
}

uint32_t pw_safetensors_count(const pw_safetensors *st) { return st ? (uint32_t)st->tensors.size() : 0u; }

int pw_safetensors_tensor(const pw_safetensors *st, const char *name, pw_tensor_info *info)
{
    if (!st || !name || !info)
        return pw::fail(PW_ERR_ARGUMENT, "null argument");
    const auto it = st->tensors.find(name);
    if (it == st->tensors.end())
        return pw::fail(PW_ERR_ARGUMENT, "tensor is absent: %s", name);
    const TensorRecord &r = it->second;
    if (r.shape.size() > 8)
        return pw::fail(PW_ERR_LAYOUT, "%s: rank above 8", name);
    memset(info, 0, sizeof *info);
    snprintf(info->dtype, sizeof info->dtype, "%s", r.dtype.c_str());
    info->rank = (uint32_t)r.shape.size();
    for (size_t i = 0; i < r.shape.size(); ++i)
        info->shape[i] = r.shape[i];
    info->region.bytes = st->map + st->payload_start + r.start;
    info->region.region_bytes = r.end - r.start;
    info->region.tensor_offset = 0;
    info->region.tensor_bytes = r.end - r.start;
    return PW_OK;
}

}  // extern "C"

namespace {

struct FoundTensor {
    const pw_safetensors *file = nullptr;
    pw_tensor_info info{};
};

bool find_tensor(const pw_safetensors *const *files, uint32_t n, const std::string &name, FoundTensor &out)
{
    for (uint32_t i = 0; i < n; ++i)
        if (files[i] && files[i]->tensors.count(name)) {
            out.file = files[i];
            return pw_safetensors_tensor(files[i], name.c_str(), &out.info) == PW_OK;
        }
    return false;
}

// validate_fp8_views_internal (src/lib.rs:1217-1270) for one projection: F8_E4M3 rank 2 of the
// expected shape (multiples of 128), F32 scale grid [rows/128, cols/128], finite scales, optionally
// no 0x7f/0xff code.
int validate_projection(const FoundTensor &w, const FoundTensor &s, const std::string &name, uint64_t rows,
                        uint64_t cols, int scan_codes)
{
    if (strcmp(w.info.dtype, "F8_E4M3") != 0 || w.info.rank != 2)
        return pw::fail(PW_ERR_LAYOUT, "%s: FP8 GEMV weight must be F8_E4M3 rank two", name.c_str());
    if (w.info.shape[0] != rows || w.info.shape[1] != cols)
        return pw::fail(PW_ERR_LAYOUT, "%s: projection shape mismatch", name.c_str());
    if (rows % 128 || cols % 128)
        return pw::fail(PW_ERR_LAYOUT, "%s: FP8 GEMV dimensions must be nonzero multiples of 128", name.c_str());
    if (strcmp(s.info.dtype, "F32") != 0 || s.info.rank != 2 || s.info.shape[0] != rows / 128 ||
        s.info.shape[1] != cols / 128)
        return pw::fail(PW_ERR_LAYOUT, "%s: FP8 GEMV scale grid mismatch", name.c_str());
    const float *sc = (const float *)s.info.region.bytes;
    for (uint64_t i = 0; i < (rows / 128) * (cols / 128); ++i) {
        float v;
        memcpy(&v, sc + i, 4);
        if (!std::isfinite(v))
            return pw::fail(PW_ERR_NONFINITE, "%s: FP8 GEMV scale is non-finite", name.c_str());
    }
    if (scan_codes) {
        const uint8_t *b = (const uint8_t *)w.info.region.bytes;
        for (uint64_t i = 0; i < rows * cols; ++i)
            if ((b[i] & 0x7f) == 0x7f)
                return pw::fail(PW_ERR_NONFINITE, "%s: non-finite FP8 weight at byte offset %llu", name.c_str(),
                                (unsigned long long)i);
    }
    return PW_OK;
}

}  // namespace

extern "C" int pw_expert_bank_from_safetensors(pw_runtime *rt, const pw_safetensors *const *files, uint32_t n_files,
                                               uint32_t layer, uint32_t n_experts, uint32_t hidden,
                                               uint32_t intermediate, int scan_codes, pw_expert_bank **out)
{
    if (!rt || !files || n_files == 0 || !out || n_experts == 0)
        return pw::fail(PW_ERR_ARGUMENT, "null argument or empty bank");
    *out = nullptr;
    if (n_experts > 1024)
        return pw::fail(PW_ERR_ARGUMENT, "a bank holds at most 1024 experts (got %u)", n_experts);
    const uint64_t H = hidden, I = intermediate;
    if (H == 0 || I == 0 || H % 128 || I % 128)
        return pw::fail(PW_ERR_LAYOUT, "hidden and intermediate sizes must be nonzero multiples of 128");
    // one device allocation: weights of every expert (gate, up, down), then their scale grids;
    // 256-byte aligned pieces
    const uint64_t wbytes[3] = {I * H, I * H, H * I};
    const uint64_t sbytes[3] = {(I / 128) * (H / 128) * 4, (I / 128) * (H / 128) * 4, (H / 128) * (I / 128) * 4};
    const uint64_t rows_of[3] = {I, I, H}, cols_of[3] = {H, H, I};
    auto align = [](uint64_t v) { return (v + 255) & ~255ull; };
    uint64_t per_expert = 0;
    for (int m = 0; m < 3; ++m)
        per_expert += align(wbytes[m]) + align(sbytes[m]);
    const char *proj_names[3] = {"gate", "up", "down"};
    std::vector<FoundTensor> found((size_t)n_experts * 6);
    for (uint32_t e = 0; e < n_experts; ++e)
        for (int m = 0; m < 3; ++m) {
            const std::string wname = "model.layers." + std::to_string(layer) + ".mlp.experts." + std::to_string(e) +
                                      "." + proj_names[m] + "_proj.weight";
            const std::string sname = wname + "_scale_inv";
            FoundTensor &w = found[(size_t)e * 6 + 2 * m], &s = found[(size_t)e * 6 + 2 * m + 1];
            if (!find_tensor(files, n_files, wname, w))
                return pw::fail(PW_ERR_LAYOUT, "tensor is absent: %s", wname.c_str());
            if (!find_tensor(files, n_files, sname, s))
                return pw::fail(PW_ERR_LAYOUT, "tensor is absent: %s", sname.c_str());
            const int st = validate_projection(w, s, wname, rows_of[m], cols_of[m], scan_codes);
            if (st != PW_OK)
                return st;
        }
    int st = pw::set_device_of(rt);
    if (st != PW_OK)
        return st;
    uint8_t *dev = nullptr;
    hipError_t he = hipMalloc(&dev, per_expert * n_experts);
    if (he != hipSuccess)
        return pw::fail(PW_ERR_NOMEM, "expert bank allocation of %llu bytes: %s",
                        (unsigned long long)(per_expert * n_experts), hipGetErrorString(he));
    std::vector<pw::ExpertPtrs> table(n_experts);
    for (uint32_t e = 0; e < n_experts && he == hipSuccess; ++e) {
        uint8_t *base = dev + per_expert * e;
        const uint8_t *wp[3];
        const float *sp[3];
        for (int m = 0; m < 3 && he == hipSuccess; ++m) {
            const FoundTensor &w = found[(size_t)e * 6 + 2 * m], &s = found[(size_t)e * 6 + 2 * m + 1];
            wp[m] = base;
            he = hipMemcpy(base, w.info.region.bytes, wbytes[m], hipMemcpyHostToDevice);
            base += align(wbytes[m]);
            sp[m] = (const float *)base;
            if (he == hipSuccess)
                he = hipMemcpy(base, s.info.region.bytes, sbytes[m], hipMemcpyHostToDevice);
            base += align(sbytes[m]);
        }
        table[e] = pw::ExpertPtrs{wp[0], sp[0], wp[1], sp[1], wp[2], sp[2]};
    }
    if (he != hipSuccess) {
        (void)hipFree(dev);
        return pw::fail(PW_ERR_DEVICE, "expert bank upload: %s", hipGetErrorString(he));
    }
    return pw::make_owned_bank(rt, table, hidden, intermediate, dev, per_expert * n_experts, out);
}
