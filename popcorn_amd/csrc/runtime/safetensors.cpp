// safetensors archives (include/popcorn_safetensors.h): the file is mapped
// read-only, its JSON header parsed and validated once, and tensors are
// copied from the mapping to host or device memory by name.
//
// Format (the published safetensors layout, which the reference reads through
// its MTLSafeTensors dependency, GemmaCLI Package.resolved: finnvoor/
// MTLSafeTensors@6f43d28): an 8-byte little-endian header length N, N bytes of
// UTF-8 JSON {"name": {"dtype": "BF16", "shape": [..], "data_offsets": [b, e]},
// ..., "__metadata__": {"key": "value"}} (space-padded), then the data buffer;
// offsets are relative to the buffer's start. A valid archive's tensors tile
// the buffer: sorted by offset they start at 0, each begins where the previous
// ends, and the last ends at the end of the file; e - b = elements * size.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <map>

#include "handles.hpp"
#include "popcorn_safetensors.h"

using namespace popcorn;

namespace {

constexpr uint64_t kMaxHeader = 100ull << 20;  // the format's header size limit

Error bad(const std::string &what) { return Error::invalidArgument("safetensors: " + what); }

// ---- a small JSON reader for the header --------------------------------------
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0;
    bool integral = false;
    uint64_t u = 0;  // value when integral and non-negative
    std::string str;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;
};

class Parser {
public:
    Parser(const char *p, size_t n) : p_(p), end_(p + n) {}

    Json document() {
        Json v = value(0);
        ws();
        if (p_ != end_) throw bad("header has trailing characters after the JSON object");
        return v;
    }

private:
    const char *p_, *end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    char peek() {
        ws();
        if (p_ >= end_) throw bad("header JSON ends early");
        return *p_;
    }
    void expect(char c) {
        if (peek() != c) throw bad(std::string("header JSON: expected '") + c + "'");
        ++p_;
    }

    Json value(int depth) {
        if (depth > 64) throw bad("header JSON nests too deeply");
        const char c = peek();
        Json v;
        if (c == '{') {
            v.kind = Json::Object;
            ++p_;
            if (peek() == '}') {
                ++p_;
                return v;
            }
            for (;;) {
                if (peek() != '"') throw bad("header JSON: object key must be a string");
                std::string key = string();
                expect(':');
                v.members.emplace_back(std::move(key), value(depth + 1));
                const char d = peek();
                ++p_;
                if (d == '}') break;
                if (d != ',') throw bad("header JSON: expected ',' or '}'");
            }
            return v;
        }
        if (c == '[') {
            v.kind = Json::Array;
            ++p_;
            if (peek() == ']') {
                ++p_;
                return v;
            }
            for (;;) {
                v.items.push_back(value(depth + 1));
                const char d = peek();
                ++p_;
                if (d == ']') break;
                if (d != ',') throw bad("header JSON: expected ',' or ']'");
            }
            return v;
        }
        if (c == '"') {
            v.kind = Json::String;
            v.str = string();
            return v;
        }
        if (literal("true")) {
            v.kind = Json::Bool;
            v.b = true;
            return v;
        }
        if (literal("false")) {
            v.kind = Json::Bool;
            return v;
        }
        if (literal("null")) return v;
        return number();
    }

    bool literal(const char *w) {
        const size_t n = std::strlen(w);
        if ((size_t)(end_ - p_) >= n && std::memcmp(p_, w, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }

    Json number() {
        Json v;
        v.kind = Json::Number;
        const char *s = p_;
        bool neg = false;
        if (p_ < end_ && *p_ == '-') {
            neg = true;
            ++p_;
        }
        uint64_t u = 0;
        bool digits = false, overflow = false;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_ - '0');
            if (u > (UINT64_MAX - d) / 10) overflow = true;
            u = u * 10 + d;
            digits = true;
            ++p_;
        }
        if (!digits) throw bad("header JSON: unexpected character");
        bool frac = false;
        if (p_ < end_ && *p_ == '.') {
            frac = true;
            ++p_;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            ++p_;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
        }
        v.num = std::strtod(std::string(s, p_).c_str(), nullptr);
        v.integral = !frac && !neg && !overflow;
        v.u = u;
        return v;
    }

    static void utf8(std::string &out, uint32_t cp) {
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

    uint32_t hex4() {
        if (end_ - p_ < 4) throw bad("header JSON: short \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else throw bad("header JSON: bad \\u escape");
        }
        return v;
    }

    std::string string() {
        expect('"');
        std::string out;
        for (;;) {
            if (p_ >= end_) throw bad("header JSON: unterminated string");
            const char c = *p_++;
            if (c == '"') break;
            if ((unsigned char)c < 0x20) throw bad("header JSON: control character in a string");
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= end_) throw bad("header JSON: unterminated escape");
            const char e = *p_++;
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
                if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                    if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') throw bad("header JSON: lone surrogate");
                    p_ += 2;
                    const uint32_t lo = hex4();
                    if (lo < 0xDC00 || lo >= 0xE000) throw bad("header JSON: bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(out, cp);
                break;
            }
            default: throw bad("header JSON: bad escape");
            }
        }
        return out;
    }
};

// safetensors dtype names -> (popcorn dtype tag or -1, element size).
struct DTypeInfo {
    const char *name;
    int32_t tag;
    int size;
};
constexpr DTypeInfo kDTypes[] = {
    {"BOOL", POPCORN_DTYPE_U8, 1},  {"U8", POPCORN_DTYPE_U8, 1},     {"I8", POPCORN_DTYPE_I8, 1},
    {"F8_E5M2", -1, 1},             {"F8_E4M3", -1, 1},              {"I16", POPCORN_DTYPE_I16, 2},
    {"U16", POPCORN_DTYPE_U16, 2},  {"F16", POPCORN_DTYPE_F16, 2},   {"BF16", POPCORN_DTYPE_BF16, 2},
    {"I32", POPCORN_DTYPE_I32, 4},  {"U32", POPCORN_DTYPE_U32, 4},   {"F32", POPCORN_DTYPE_F32, 4},
    {"F64", -1, 8},                 {"I64", POPCORN_DTYPE_I64, 8},   {"U64", POPCORN_DTYPE_U64, 8},
};

struct Entry {
    std::string name;
    std::string dtypeName;
    int32_t dtype = -1;
    int elemSize = 1;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
};

}  // namespace

struct popcorn_safetensors_s {
    int fd = -1;
    void *map = nullptr;
    size_t fileSize = 0;
    uint64_t dataStart = 0;
    std::vector<Entry> entries;            // header order
    std::map<std::string, size_t> byName;  // -> index in entries
    std::vector<std::pair<std::string, std::string>> metadata;

    ~popcorn_safetensors_s() {
        if (map && map != MAP_FAILED) munmap(map, fileSize);
        if (fd >= 0) close(fd);
    }

    const uint8_t *data(const Entry &e) const { return static_cast<const uint8_t *>(map) + dataStart + e.begin; }

    const Entry &find(const char *name) const {
        auto it = byName.find(name);
        if (it == byName.end()) throw bad(std::string("no tensor named \"") + name + "\"");
        return entries[it->second];
    }

    void parse() {
        if (fileSize < 8) throw bad("file shorter than the 8-byte header length");
        uint64_t n = 0;
        std::memcpy(&n, map, 8);  // little-endian host
        if (n > kMaxHeader) throw bad("header length above the format's 100 MB limit");
        if (n > fileSize - 8) throw bad("header length runs past the end of the file");
        dataStart = 8 + n;
        const uint64_t bufSize = fileSize - dataStart;
        Json root = Parser(static_cast<const char *>(map) + 8, (size_t)n).document();
        if (root.kind != Json::Object) throw bad("header is not a JSON object");
        for (auto &m : root.members) {
            if (m.first == "__metadata__") {
                if (m.second.kind != Json::Object) throw bad("__metadata__ is not an object");
                for (auto &kv : m.second.members) {
                    if (kv.second.kind != Json::String) throw bad("__metadata__ values must be strings");
                    metadata.emplace_back(kv.first, kv.second.str);
                }
                continue;
            }
            const Json &t = m.second;
            if (t.kind != Json::Object) throw bad("entry \"" + m.first + "\" is not an object");
            const Json *dt = nullptr, *shape = nullptr, *offs = nullptr;
            for (auto &f : t.members) {
                if (f.first == "dtype") dt = &f.second;
                else if (f.first == "shape") shape = &f.second;
                else if (f.first == "data_offsets") offs = &f.second;
            }
            if (!dt || dt->kind != Json::String || !shape || shape->kind != Json::Array || !offs ||
                offs->kind != Json::Array || offs->items.size() != 2)
                throw bad("entry \"" + m.first + "\" needs dtype, shape and data_offsets [begin, end]");
            Entry e;
            e.name = m.first;
            e.dtypeName = dt->str;
            const DTypeInfo *info = nullptr;
            for (const auto &d : kDTypes)
                if (e.dtypeName == d.name) info = &d;
            if (!info) throw bad("entry \"" + m.first + "\" has unknown dtype " + e.dtypeName);
            e.dtype = info->tag;
            e.elemSize = info->size;
            if (shape->items.size() > POPCORN_MAX_RANK) throw bad("entry \"" + m.first + "\" has rank above 8");
            uint64_t count = 1;
            for (const auto &d : shape->items) {
                if (d.kind != Json::Number || !d.integral || d.u > (uint64_t)INT64_MAX)
                    throw bad("entry \"" + m.first + "\" has a shape entry that is not a non-negative integer");
                if (d.u && count > UINT64_MAX / d.u) throw bad("entry \"" + m.first + "\" element count overflows");
                count *= d.u;
                e.shape.push_back((int64_t)d.u);
            }
            for (const auto &o : offs->items)
                if (o.kind != Json::Number || !o.integral) throw bad("entry \"" + m.first + "\" has a bad data offset");
            e.begin = offs->items[0].u;
            e.end = offs->items[1].u;
            if (e.begin > e.end || e.end > bufSize)
                throw bad("entry \"" + m.first + "\" data_offsets fall outside the data buffer");
            if (count > UINT64_MAX / (uint64_t)e.elemSize || e.end - e.begin != count * (uint64_t)e.elemSize)
                throw bad("entry \"" + m.first + "\" holds " + std::to_string(e.end - e.begin) + " bytes, not elements x " +
                          std::to_string(e.elemSize));
            if (byName.count(e.name)) throw bad("duplicate entry \"" + e.name + "\"");
            byName[e.name] = entries.size();
            entries.push_back(std::move(e));
        }
        // the tensors tile the buffer
        std::vector<const Entry *> order;
        for (const auto &e : entries) order.push_back(&e);
        std::sort(order.begin(), order.end(), [](const Entry *a, const Entry *b) {
            return a->begin != b->begin ? a->begin < b->begin : a->end < b->end;
        });
        uint64_t at = 0;
        for (const Entry *e : order) {
            if (e->begin != at) throw bad("data_offsets of \"" + e->name + "\" leave a hole or overlap another tensor");
            at = e->end;
        }
        if (at != bufSize) throw bad("the data buffer has bytes no tensor covers");
    }
};

namespace {

popcorn_status_t guardedSt(const std::function<void()> &f) {
    try {
        f();
        setLastError("");
        return POPCORN_OK;
    } catch (const Error &e) {
        setLastError(e.what());
        return e.code();
    } catch (const std::exception &e) {
        setLastError(e.what());
        return POPCORN_ERR_GPU_INTERNAL;
    }
}

void fill(popcorn_safetensors_info_t *info, const Entry &e, int32_t index) {
    std::memset(info, 0, sizeof(*info));
    std::strncpy(info->name, e.name.c_str(), sizeof(info->name) - 1);
    std::strncpy(info->dtype_name, e.dtypeName.c_str(), sizeof(info->dtype_name) - 1);
    info->dtype = e.dtype;
    info->rank = (int32_t)e.shape.size();
    for (size_t i = 0; i < e.shape.size(); ++i) info->shape[i] = e.shape[i];
    info->offset = e.begin;
    info->nbytes = e.end - e.begin;
    info->index = index;
}

const Entry &readable(popcorn_safetensors_t a, const char *name, size_t capacity) {
    if (!a || !name) throw Error::invalidArgument("archive and name must not be NULL");
    const Entry &e = a->find(name);
    if (e.dtype < 0)
        throw Error::unsupportedDataTypeCombination("safetensors dtype " + e.dtypeName + " of \"" + e.name +
                                                    "\" has no tensor data type here");
    if (capacity < e.end - e.begin)
        throw Error::invalidArgument("destination holds " + std::to_string(capacity) + " bytes; \"" + e.name + "\" has " +
                                     std::to_string(e.end - e.begin));
    return e;
}

}  // namespace

extern "C" {

popcorn_status_t popcorn_safetensors_open(const char *path, popcorn_safetensors_t *archive) {
    return guardedSt([&] {
        if (!path || !archive) throw Error::invalidArgument("path and archive must not be NULL");
        auto a = std::make_unique<popcorn_safetensors_s>();
        a->fd = open(path, O_RDONLY | O_CLOEXEC);
        if (a->fd < 0) throw Error::invalidArgument(std::string("cannot open ") + path + ": " + std::strerror(errno));
        struct stat st {};
        if (fstat(a->fd, &st) != 0) throw Error::invalidArgument(std::string("cannot stat ") + path);
        a->fileSize = (size_t)st.st_size;
        if (a->fileSize) {
            a->map = mmap(nullptr, a->fileSize, PROT_READ, MAP_PRIVATE, a->fd, 0);
            if (a->map == MAP_FAILED) {
                a->map = nullptr;
                throw Error::invalidArgument(std::string("cannot map ") + path);
            }
        }
        a->parse();
        *archive = a.release();
    });
}

popcorn_status_t popcorn_safetensors_close(popcorn_safetensors_t archive) {
    return guardedSt([&] { delete archive; });
}

int32_t popcorn_safetensors_count(popcorn_safetensors_t archive) {
    return archive ? (int32_t)archive->entries.size() : 0;
}

popcorn_status_t popcorn_safetensors_info(popcorn_safetensors_t archive, int32_t index, popcorn_safetensors_info_t *info) {
    return guardedSt([&] {
        if (!archive || !info) throw Error::invalidArgument("archive and info must not be NULL");
        if (index < 0 || (size_t)index >= archive->entries.size()) throw Error::invalidArgument("tensor index out of range");
        fill(info, archive->entries[(size_t)index], index);
    });
}

popcorn_status_t popcorn_safetensors_find(popcorn_safetensors_t archive, const char *name, popcorn_safetensors_info_t *info) {
    return guardedSt([&] {
        if (!archive || !name || !info) throw Error::invalidArgument("archive, name and info must not be NULL");
        const Entry &e = archive->find(name);
        fill(info, e, (int32_t)archive->byName.at(name));
    });
}

popcorn_status_t popcorn_safetensors_metadata(popcorn_safetensors_t archive, const char *key, char *value, size_t capacity) {
    return guardedSt([&] {
        if (!archive || !key || !value || !capacity) throw Error::invalidArgument("archive, key and value must not be NULL");
        for (const auto &kv : archive->metadata) {
            if (kv.first == key) {
                if (kv.second.size() + 1 > capacity) throw Error::invalidArgument("metadata value longer than the buffer");
                std::memcpy(value, kv.second.c_str(), kv.second.size() + 1);
                return;
            }
        }
        throw Error::invalidArgument(std::string("no metadata key \"") + key + "\"");
    });
}

popcorn_status_t popcorn_safetensors_read(popcorn_safetensors_t archive, const char *name, void *dst, size_t capacity) {
    return guardedSt([&] {
        const Entry &e = readable(archive, name, capacity);
        if (e.end > e.begin) {
            if (!dst) throw Error::invalidArgument("destination must not be NULL");
            std::memcpy(dst, archive->data(e), e.end - e.begin);
        }
    });
}

popcorn_status_t popcorn_safetensors_upload(popcorn_safetensors_t archive, const char *name, void *device_dst, size_t capacity,
                                            popcorn_stream_t stream) {
    return guardedSt([&] {
        const Entry &e = readable(archive, name, capacity);
        if (e.end == e.begin) return;
        if (!device_dst) throw Error::invalidArgument("destination must not be NULL");
        hipStream_t s = reinterpret_cast<hipStream_t>(stream);
        // from pageable mapped memory: the copy has read the mapping when the
        // stream is synchronized
        checkHip(hipMemcpyAsync(device_dst, archive->data(e), e.end - e.begin, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
        checkHip(hipStreamSynchronize(s), "hipStreamSynchronize");
    });
}

}  // extern "C"
