// Kernel parameter layouts read from the code objects themselves.
//
// A gfx950 code object (an ELF, or a clang offload bundle holding one) carries
// the AMDGPU metadata note (NT_AMDGPU_METADATA, a MessagePack map): for every
// kernel, `.name` and `.args`, each argument with `.size`, `.offset` and
// `.value_kind` (`global_buffer` for a device pointer, `by_value` for a
// constants block, `hidden_*` for what the runtime appends). The explicit
// arguments are the kernel's parameter list, which a raw launch must match:
// the reference binds the tensors, then each constants block
// (KernelCommandEncoder.swift:199-204), and a launch whose pointer count or
// block sizes differ from the kernel's would read past the caller's arrays.
#include <cstring>
#include <fstream>
#include <iterator>

#include "popcorn.hpp"

namespace popcorn {
namespace {

// ---- a minimal MessagePack reader (the subset the metadata uses) ----------

struct MpValue {
    enum Kind { Nil, Bool, Int, Float, Str, Arr, Map } kind = Nil;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    std::vector<MpValue> arr;
    std::vector<std::pair<MpValue, MpValue>> map;

    const MpValue *get(const char *key) const {
        if (kind != Map) return nullptr;
        for (const auto &kv : map)
            if (kv.first.kind == Str && kv.first.s == key) return &kv.second;
        return nullptr;
    }
};

class MpReader {
public:
    MpReader(const uint8_t *p, size_t n) : p_(p), end_(p + n) {}

    MpValue read(int depth = 0) {
        if (depth > 32) fail("nesting too deep");
        const uint8_t t = byte();
        MpValue v;
        if (t <= 0x7f) return integer(t);
        if (t >= 0xe0) return integer((int8_t)t);
        if ((t & 0xf0) == 0x80) return mapOf(t & 0x0f, depth);
        if ((t & 0xf0) == 0x90) return arrayOf(t & 0x0f, depth);
        if ((t & 0xe0) == 0xa0) return str(t & 0x1f);
        switch (t) {
        case 0xc0: return v;
        case 0xc2: v.kind = MpValue::Bool; v.i = 0; return v;
        case 0xc3: v.kind = MpValue::Bool; v.i = 1; return v;
        case 0xc4: skip(be(1)); return v;  // bin: not used by the metadata
        case 0xc5: skip(be(2)); return v;
        case 0xc6: skip(be(4)); return v;
        case 0xca: {
            uint32_t b = (uint32_t)be(4);
            float x;
            std::memcpy(&x, &b, 4);
            v.kind = MpValue::Float;
            v.f = x;
            return v;
        }
        case 0xcb: {
            uint64_t b = be(8);
            double x;
            std::memcpy(&x, &b, 8);
            v.kind = MpValue::Float;
            v.f = x;
            return v;
        }
        case 0xcc: return integer((int64_t)be(1));
        case 0xcd: return integer((int64_t)be(2));
        case 0xce: return integer((int64_t)be(4));
        case 0xcf: return integer((int64_t)be(8));
        case 0xd0: return integer((int8_t)be(1));
        case 0xd1: return integer((int16_t)be(2));
        case 0xd2: return integer((int32_t)be(4));
        case 0xd3: return integer((int64_t)be(8));
        case 0xd9: return str(be(1));
        case 0xda: return str(be(2));
        case 0xdb: return str(be(4));
        case 0xdc: return arrayOf(be(2), depth);
        case 0xdd: return arrayOf(be(4), depth);
        case 0xde: return mapOf(be(2), depth);
        case 0xdf: return mapOf(be(4), depth);
        default: fail("unsupported type byte " + std::to_string(t));
        }
        return v;
    }

private:
    [[noreturn]] static void fail(const std::string &why) {
        throw Error::invalidArgument("malformed code object metadata: " + why);
    }
    uint8_t byte() {
        if (p_ >= end_) fail("truncated");
        return *p_++;
    }
    uint64_t be(int n) {
        uint64_t v = 0;
        for (int i = 0; i < n; ++i) v = (v << 8) | byte();
        return v;
    }
    void skip(uint64_t n) {
        if (n > (uint64_t)(end_ - p_)) fail("truncated");
        p_ += n;
    }
    static MpValue integer(int64_t x) {
        MpValue v;
        v.kind = MpValue::Int;
        v.i = x;
        return v;
    }
    MpValue str(uint64_t n) {
        if (n > (uint64_t)(end_ - p_)) fail("truncated string");
        MpValue v;
        v.kind = MpValue::Str;
        v.s.assign(reinterpret_cast<const char *>(p_), (size_t)n);
        p_ += n;
        return v;
    }
    MpValue arrayOf(uint64_t n, int depth) {
        if (n > (uint64_t)(end_ - p_)) fail("array longer than the note");
        MpValue v;
        v.kind = MpValue::Arr;
        for (uint64_t k = 0; k < n; ++k) v.arr.push_back(read(depth + 1));
        return v;
    }
    MpValue mapOf(uint64_t n, int depth) {
        if (n > (uint64_t)(end_ - p_)) fail("map longer than the note");
        MpValue v;
        v.kind = MpValue::Map;
        for (uint64_t k = 0; k < n; ++k) {
            MpValue key = read(depth + 1);
            MpValue val = read(depth + 1);
            v.map.emplace_back(std::move(key), std::move(val));
        }
        return v;
    }

    const uint8_t *p_;
    const uint8_t *end_;
};

template <typename T>
T rd(const std::vector<uint8_t> &b, size_t off) {
    if (off + sizeof(T) > b.size()) throw Error::invalidArgument("malformed code object: truncated header");
    T v;
    std::memcpy(&v, b.data() + off, sizeof(T));
    return v;
}

bool isElf64(const uint8_t *p, size_t n) {
    return n >= 64 && p[0] == 0x7f && p[1] == 'E' && p[2] == 'L' && p[3] == 'F' && p[4] == 2 && p[5] == 1;
}

// The AMDGPU ELF inside a clang offload bundle (magic, entry count, then per
// entry offset, size, triple length, triple); the file itself if it is an ELF.
std::vector<uint8_t> amdgpuElf(const std::vector<uint8_t> &file) {
    static const char kMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
    const size_t ml = sizeof(kMagic) - 1;
    if (isElf64(file.data(), file.size())) return file;
    if (file.size() < ml + 8 || std::memcmp(file.data(), kMagic, ml) != 0)
        throw Error::invalidArgument("code object is neither an ELF nor an offload bundle");
    const uint64_t n = rd<uint64_t>(file, ml);
    size_t at = ml + 8;
    for (uint64_t e = 0; e < n && e < 1024; ++e) {
        const uint64_t off = rd<uint64_t>(file, at), size = rd<uint64_t>(file, at + 8), tl = rd<uint64_t>(file, at + 16);
        at += 24;
        if (tl > file.size() - at) throw Error::invalidArgument("malformed offload bundle entry");
        const std::string triple(reinterpret_cast<const char *>(file.data() + at), (size_t)tl);
        at += (size_t)tl;
        if (triple.find("amdgcn") == std::string::npos) continue;
        if (off > file.size() || size > file.size() - off) throw Error::invalidArgument("malformed offload bundle entry");
        if (isElf64(file.data() + off, (size_t)size)) return std::vector<uint8_t>(file.begin() + (long)off, file.begin() + (long)(off + size));
    }
    throw Error::invalidArgument("offload bundle holds no amdgcn ELF");
}

}  // namespace

std::map<std::string, KernelLayout> readKernelLayouts(const std::vector<uint8_t> &file) {
    const std::vector<uint8_t> elf = amdgpuElf(file);
    const uint64_t shoff = rd<uint64_t>(elf, 0x28);
    const uint16_t shentsize = rd<uint16_t>(elf, 0x3a), shnum = rd<uint16_t>(elf, 0x3c);
    std::map<std::string, KernelLayout> out;
    bool found = false;
    for (uint16_t i = 0; i < shnum; ++i) {
        const size_t sh = (size_t)shoff + (size_t)i * shentsize;
        if (rd<uint32_t>(elf, sh + 4) != 7u) continue;  // SHT_NOTE
        const uint64_t off = rd<uint64_t>(elf, sh + 0x18), size = rd<uint64_t>(elf, sh + 0x20);
        if (off > elf.size() || size > elf.size() - off) throw Error::invalidArgument("malformed code object note section");
        size_t at = (size_t)off;
        const size_t end = (size_t)(off + size);
        while (at + 12 <= end) {
            const uint32_t namesz = rd<uint32_t>(elf, at), descsz = rd<uint32_t>(elf, at + 4), type = rd<uint32_t>(elf, at + 8);
            const size_t name = at + 12, desc = name + ((namesz + 3u) & ~3u);
            if (desc > end || descsz > end - desc) throw Error::invalidArgument("malformed code object note");
            at = desc + ((descsz + 3u) & ~3u);
            if (type != 32u || namesz < 6 || std::memcmp(elf.data() + name, "AMDGPU", 6) != 0) continue;
            MpReader r(elf.data() + desc, descsz);
            const MpValue root = r.read();
            const MpValue *kernels = root.get("amdhsa.kernels");
            if (!kernels || kernels->kind != MpValue::Arr) continue;
            found = true;
            for (const MpValue &k : kernels->arr) {
                const MpValue *nm = k.get(".name");
                if (!nm || nm->kind != MpValue::Str) continue;
                KernelLayout L;
                if (const MpValue *a = k.get(".args"); a && a->kind == MpValue::Arr) {
                    for (const MpValue &arg : a->arr) {
                        const MpValue *kind = arg.get(".value_kind"), *sz = arg.get(".size"), *ofs = arg.get(".offset");
                        if (!kind || kind->kind != MpValue::Str || !sz || sz->kind != MpValue::Int) continue;
                        if (kind->s.rfind("hidden_", 0) == 0) continue;
                        KernelArg ka;
                        ka.pointer = kind->s == "global_buffer" || kind->s == "dynamic_shared_pointer";
                        ka.size = (uint32_t)sz->i;
                        ka.offset = ofs && ofs->kind == MpValue::Int ? (uint32_t)ofs->i : 0u;
                        L.args.push_back(ka);
                    }
                }
                if (const MpValue *v = k.get(".kernarg_segment_size"); v && v->kind == MpValue::Int) L.kernargBytes = (uint32_t)v->i;
                if (const MpValue *v = k.get(".max_flat_workgroup_size"); v && v->kind == MpValue::Int)
                    L.maxThreads = (uint32_t)v->i;
                if (const MpValue *v = k.get(".group_segment_fixed_size"); v && v->kind == MpValue::Int)
                    L.staticLds = (uint32_t)v->i;
                out[nm->s] = std::move(L);
            }
        }
    }
    if (!found) throw Error::invalidArgument("code object has no AMDGPU kernel metadata");
    return out;
}

std::map<std::string, KernelLayout> readKernelLayouts(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error::invalidArgument("cannot open code object " + path);
    std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    return readKernelLayouts(bytes);
}

std::string KernelLayout::str() const {
    int nptr = 0;
    while (nptr < (int)args.size() && args[(size_t)nptr].pointer) ++nptr;
    std::string s = std::to_string(nptr) + " device pointers";
    for (size_t i = (size_t)nptr; i < args.size(); ++i) {
        s += i == (size_t)nptr ? ", then " : ", ";
        s += args[i].pointer ? "a device pointer" : "a " + std::to_string(args[i].size) + "-byte constants block";
    }
    return s;
}

void KernelLayout::check(const std::string &name, size_t nbuffers, const std::vector<size_t> &constantSizes) const {
    bool ok = nbuffers + constantSizes.size() == args.size();
    for (size_t i = 0; ok && i < args.size(); ++i) {
        if (i < nbuffers) ok = args[i].pointer;
        else ok = !args[i].pointer && args[i].size == constantSizes[i - nbuffers];
    }
    if (ok) return;
    std::string got = std::to_string(nbuffers) + " device pointers";
    for (size_t j = 0; j < constantSizes.size(); ++j)
        got += (j ? ", " : ", then ") + std::string("a ") + std::to_string(constantSizes[j]) + "-byte constants block";
    throw Error::invalidArgument("launch of " + name + " does not match its parameter list: the kernel takes " + str() +
                                 "; the launch binds " + got + ".");
}

}  // namespace popcorn
