/*
 * g4s_store.hip -- the engine's weight store on the host: a VPK archive
 * (TVFS, src/vendor/StdApp/StdApp.VFS.pas) holding a JSON manifest and one
 * weights file (TWeightStore, src/Gemma4.Tensors.pas:321-506), and the
 * upload of a Q4_0 tensor -- the tied embedding / LM head weight -- into
 * device memory in the sampler's layouts.
 *
 * Archive layout (StdApp.VFS.pas:68-84, packed little-endian records):
 *   header  52 bytes: magic "VPK0", version UInt32 = 1, entry count UInt32,
 *           data start UInt64, 32 reserved bytes;
 *   entries 544 bytes each, directly after the header: path as 260 UTF-16
 *           code units (NUL-terminated when shorter), offset UInt64 (from
 *           the start of the archive), size UInt64, CRC-32 UInt32, flags
 *           UInt32;
 *   data    the entries' bytes.
 * The archive is memory-mapped read-only, as TVFS.Open does (:243-332),
 * with the same checks in the same order (size >= header, magic, version,
 * size >= header + directory).  Lookups normalise the requested path the way
 * TVFS.NormalizePath does (:180-183: '\' -> '/', lower case; the lower-casing
 * here covers ASCII, which is what the engine's archives hold); the stored
 * entry paths are used as written, as the reference does (:316-323).
 */
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "gemma4_sampler.h"
#include "g4s_lmhead.h"
#include "g4s_runtime.h"

#define G4S_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr uint32_t kVpkVersion = 1;          /* VFS_VERSION, StdApp.VFS.pas:51 */
constexpr size_t kHeaderBytes = 4 + 4 + 4 + 8 + 32;
constexpr size_t kPathUnits = 260;
constexpr size_t kEntryBytes = kPathUnits * 2 + 8 + 8 + 4 + 4;
static_assert(kHeaderBytes == 52 && kEntryBytes == 544, "packed VPK records");

template <typename T>
T rd(const uint8_t* p)
{
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

struct Entry {
    std::string path; /* UTF-8 */
    uint64_t offset = 0, size = 0;
    uint32_t crc = 0, flags = 0;
};

/* ------------------------------------------------------------------ JSON */

/* A JSON value: enough of the grammar (RFC 8259) for the manifest. */
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    bool is_int = false;   /* the number was written without fraction or exponent */
    bool negative = false;
    uint64_t u = 0;        /* |integer| when is_int and it fits */
    std::string s;
    std::vector<JVal> items;
    std::vector<std::pair<std::string, JVal>> members;

    const JVal* get(const char* key) const
    {
        if (kind != Obj) return nullptr;
        const JVal* hit = nullptr;
        for (const auto& m : members)
            if (m.first == key) hit = &m.second; /* the last duplicate wins */
        return hit;
    }
};

class JParser {
  public:
    JParser(const char* p, const char* e) : p_(p), e_(e) {}

    bool parse(JVal& out)
    {
        ws();
        if (!value(out, 0)) return false;
        ws();
        return p_ == e_;
    }
    const char* where() const { return p_; }

  private:
    const char* p_;
    const char* e_;

    void ws()
    {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w)
    {
        const size_t n = std::strlen(w);
        if ((size_t)(e_ - p_) < n || std::memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void put_utf8(std::string& s, uint32_t c)
    {
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xC0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += (char)(0xE0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        } else {
            s += (char)(0xF0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3F));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t& v)
    {
        if (e_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s)
    {
        if (p_ >= e_ || *p_ != '"') return false;
        ++p_;
        while (p_ < e_ && *p_ != '"') {
            const unsigned char c = (unsigned char)*p_;
            if (c < 0x20) return false;
            if (c != '\\') {
                s += (char)c;
                ++p_;
                continue;
            }
            if (++p_ >= e_) return false;
            const char esc = *p_++;
            switch (esc) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                uint32_t c1;
                if (!hex4(c1)) return false;
                if (c1 >= 0xD800 && c1 < 0xDC00 && e_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                    const char* save = p_;
                    p_ += 2;
                    uint32_t c2;
                    if (hex4(c2) && c2 >= 0xDC00 && c2 < 0xE000)
                        c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                    else
                        p_ = save;
                }
                put_utf8(s, c1);
                break;
            }
            default: return false;
            }
        }
        if (p_ >= e_) return false;
        ++p_;
        return true;
    }
    bool number(JVal& v)
    {
        const char* b = p_;
        if (p_ < e_ && *p_ == '-') ++p_;
        const char* d0 = p_;
        while (p_ < e_ && std::isdigit((unsigned char)*p_)) ++p_;
        if (p_ == d0) return false;
        bool frac = false;
        if (p_ < e_ && *p_ == '.') {
            frac = true;
            ++p_;
            const char* f0 = p_;
            while (p_ < e_ && std::isdigit((unsigned char)*p_)) ++p_;
            if (p_ == f0) return false;
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            ++p_;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
            const char* x0 = p_;
            while (p_ < e_ && std::isdigit((unsigned char)*p_)) ++p_;
            if (p_ == x0) return false;
        }
        const std::string txt(b, p_);
        v.kind = JVal::Num;
        v.num = std::strtod(txt.c_str(), nullptr);
        v.negative = *b == '-';
        v.is_int = !frac;
        if (v.is_int) {
            uint64_t acc = 0;
            bool fits = true;
            for (const char* q = d0; q < p_; ++q) {
                const uint64_t dgt = (uint64_t)(*q - '0');
                if (acc > (UINT64_MAX - dgt) / 10) fits = false;
                acc = acc * 10 + dgt;
            }
            v.u = acc;
            if (!fits) v.is_int = false;
        }
        return true;
    }
    bool value(JVal& v, int depth)
    {
        if (depth > 64 || p_ >= e_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = JVal::Obj;
            ws();
            if (p_ < e_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p_ >= e_ || *p_ != ':') return false;
                ++p_;
                ws();
                JVal m;
                if (!value(m, depth + 1)) return false;
                v.members.emplace_back(std::move(k), std::move(m));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = JVal::Arr;
            ws();
            if (p_ < e_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                JVal m;
                if (!value(m, depth + 1)) return false;
                v.items.push_back(std::move(m));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v.kind = JVal::Str;
            return string(v.s);
        }
        if (lit("true")) {
            v.kind = JVal::Bool;
            v.b = true;
            return true;
        }
        if (lit("false")) {
            v.kind = JVal::Bool;
            return true;
        }
        if (lit("null")) return true;
        return number(v);
    }
};

/* TJSON accessors with the reference's defaults (AsString(''), AsUInt64(0),
 * AsInt32(0)): a missing or differently typed value gives the default. */
std::string as_string(const JVal* v) { return v && v->kind == JVal::Str ? v->s : std::string(); }

uint64_t as_u64(const JVal* v)
{
    if (!v || v->kind != JVal::Num || !v->is_int || v->negative) return 0;
    return v->u;
}

int32_t as_i32(const JVal* v)
{
    if (!v || v->kind != JVal::Num || !v->is_int || v->u > 0x7FFFFFFFull) return 0;
    return v->negative ? -(int32_t)v->u : (int32_t)v->u;
}

/* DtypeKindFromString, src/Gemma4.Types.pas:505-517 (exact, case-sensitive). */
int32_t dtype_kind(const std::string& s)
{
    if (s == "BF16") return G4S_WDTYPE_BF16;
    if (s == "F16") return G4S_WDTYPE_F16;
    if (s == "F32") return G4S_WDTYPE_F32;
    if (s == "Q4_0") return G4S_WDTYPE_Q4_0;
    return G4S_WDTYPE_UNKNOWN;
}

std::string utf16_to_utf8(const uint8_t* p, size_t units)
{
    std::string s;
    for (size_t i = 0; i < units; ++i) {
        uint32_t c = rd<uint16_t>(p + 2 * i);
        if (c >= 0xD800 && c < 0xDC00 && i + 1 < units) {
            const uint32_t c2 = rd<uint16_t>(p + 2 * (i + 1));
            if (c2 >= 0xDC00 && c2 < 0xE000) {
                c = 0x10000 + ((c - 0xD800) << 10) + (c2 - 0xDC00);
                ++i;
            }
        }
        if (c < 0x80) {
            s += (char)c;
        } else if (c < 0x800) {
            s += (char)(0xC0 | (c >> 6));
            s += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            s += (char)(0xE0 | (c >> 12));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        } else {
            s += (char)(0xF0 | (c >> 18));
            s += (char)(0x80 | ((c >> 12) & 0x3F));
            s += (char)(0x80 | ((c >> 6) & 0x3F));
            s += (char)(0x80 | (c & 0x3F));
        }
    }
    return s;
}

/* TVFS.NormalizePath, StdApp.VFS.pas:180-183. */
std::string normalize_path(const char* path)
{
    std::string s(path);
    for (auto& c : s) {
        if (c == '\\') c = '/';
        else if (c >= 'A' && c <= 'Z') c = (char)(c - 'A' + 'a');
    }
    return s;
}

/* TPath.ChangeExtension(AFilename, 'vpk') as TVFS.Open applies it (:255):
 * the extension of the last path component is replaced, or added. */
std::string vpk_filename(const char* path)
{
    std::string s(path);
    const size_t slash = s.find_last_of('/');
    const size_t dot = s.find_last_of('.');
    if (dot != std::string::npos && (slash == std::string::npos || dot > slash))
        s.resize(dot);
    return s + ".vpk";
}

/* CRC-32 of TVFS.ComputeCRC32 (:185-198): reflected polynomial 0xEDB88320,
 * initial value and final xor 0xFFFFFFFF (the common CRC-32 of zlib). */
uint32_t crc32_bytes(const uint8_t* p, uint64_t n)
{
    static uint32_t table[256];
    static bool init = false;
    if (!init) {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int k = 0; k < 8; ++k) c = (c & 1u) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
            table[i] = c;
        }
        init = true;
    }
    uint32_t c = 0xFFFFFFFFu;
    for (uint64_t i = 0; i < n; ++i) c = table[(c ^ p[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

thread_local std::string g_open_error;

}  // namespace

struct g4s_store {
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t bytes = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> lookup;
    std::vector<std::string> names;        /* manifest order */
    std::vector<g4s_tensor_info> infos;
    std::unordered_map<std::string, size_t> tensor_lookup;
    size_t weights_entry = 0;
    std::string err;
};

namespace {

int store_fail(g4s_store* st, int code, const char* fmt, ...)
{
    char buf[768];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (st)
        st->err = buf;
    else
        g_open_error = buf;
    return code;
}

void store_release(g4s_store* st)
{
    if (st->base) munmap(const_cast<uint8_t*>(st->base), st->bytes);
    if (st->fd >= 0) close(st->fd);
    st->base = nullptr;
    st->fd = -1;
}

const Entry* find_entry(const g4s_store* st, const char* path)
{
    const auto it = st->lookup.find(normalize_path(path));
    return it == st->lookup.end() ? nullptr : &st->entries[it->second];
}

/* TVFS.Open, StdApp.VFS.pas:243-332. */
int vfs_open(g4s_store* st, const std::string& file)
{
    st->fd = open(file.c_str(), O_RDONLY | O_CLOEXEC);
    if (st->fd < 0)
        return store_fail(nullptr, G4S_ERR_IO, "Failed to open VPK: %s (%s)", file.c_str(),
                          std::strerror(errno));
    struct stat sb;
    if (fstat(st->fd, &sb) != 0 || !S_ISREG(sb.st_mode))
        return store_fail(nullptr, G4S_ERR_IO, "Failed to open VPK: %s (not a regular file)",
                          file.c_str());
    st->bytes = (uint64_t)sb.st_size;
    if (st->bytes < kHeaderBytes)
        return store_fail(nullptr, G4S_ERR_FORMAT, "VPK truncated: %llu bytes, header needs %zu",
                          (unsigned long long)st->bytes, kHeaderBytes);
    void* m = mmap(nullptr, st->bytes, PROT_READ, MAP_PRIVATE, st->fd, 0);
    if (m == MAP_FAILED)
        return store_fail(nullptr, G4S_ERR_IO, "Failed to map VPK: %s (%s)", file.c_str(),
                          std::strerror(errno));
    st->base = static_cast<const uint8_t*>(m);
    if (std::memcmp(st->base, "VPK0", 4) != 0)
        return store_fail(nullptr, G4S_ERR_FORMAT, "Invalid VPK magic");
    const uint32_t version = rd<uint32_t>(st->base + 4);
    if (version != kVpkVersion)
        return store_fail(nullptr, G4S_ERR_FORMAT, "Unsupported VPK version: %u", version);
    const uint32_t count = rd<uint32_t>(st->base + 8);
    if (st->bytes < kHeaderBytes + (uint64_t)count * kEntryBytes)
        return store_fail(nullptr, G4S_ERR_FORMAT, "VPK truncated: directory of %u entries", count);
    st->entries.resize(count);
    for (uint32_t i = 0; i < count; ++i) {
        const uint8_t* e = st->base + kHeaderBytes + (size_t)i * kEntryBytes;
        size_t len = 0;
        while (len < kPathUnits && rd<uint16_t>(e + 2 * len) != 0) ++len;
        Entry& en = st->entries[i];
        en.path = utf16_to_utf8(e, len);
        en.offset = rd<uint64_t>(e + kPathUnits * 2);
        en.size = rd<uint64_t>(e + kPathUnits * 2 + 8);
        en.crc = rd<uint32_t>(e + kPathUnits * 2 + 16);
        en.flags = rd<uint32_t>(e + kPathUnits * 2 + 20);
        st->lookup[en.path] = i; /* AddOrSetValue: a later duplicate wins */
    }
    return G4S_OK;
}

/* The bytes of an entry (TVFS.OpenFile, :348-363), range-checked against the
 * archive; a failure is reported on `target` (NULL: the thread's open error). */
int entry_view(const g4s_store* st, const Entry& en, const uint8_t** p, g4s_store* target)
{
    if (en.offset > st->bytes || en.size > st->bytes - en.offset)
        return store_fail(target, G4S_ERR_FORMAT,
                          "VPK entry %s [%llu, +%llu) lies beyond the archive (%llu bytes)",
                          en.path.c_str(), (unsigned long long)en.offset,
                          (unsigned long long)en.size, (unsigned long long)st->bytes);
    *p = st->base + en.offset;
    return G4S_OK;
}

/* TWeightStore.DoParseManifest, src/Gemma4.Tensors.pas:396-455. */
int parse_manifest(g4s_store* st, const uint8_t* p, uint64_t n)
{
    JVal root;
    JParser jp(reinterpret_cast<const char*>(p), reinterpret_cast<const char*>(p) + n);
    if (!jp.parse(root))
        return store_fail(nullptr, G4S_ERR_FORMAT,
                          "Failed to parse manifest JSON (byte %lld)",
                          (long long)(jp.where() - reinterpret_cast<const char*>(p)));
    const JVal* tensors = root.get("tensors");
    if (!tensors || tensors->kind == JVal::Null)
        return store_fail(nullptr, G4S_ERR_FORMAT, "Missing tensors array in manifest");
    if (tensors->kind == JVal::Arr) {
        for (const JVal& it : tensors->items) {
            g4s_tensor_info info{};
            const std::string name = as_string(it.get("name"));
            info.source_dtype = dtype_kind(as_string(it.get("source_dtype")));
            info.output_dtype = dtype_kind(as_string(it.get("output_dtype")));
            info.offset = as_u64(it.get("offset"));
            info.size = as_u64(it.get("size"));
            const JVal* shape = it.get("shape");
            if (shape && shape->kind == JVal::Arr) {
                if (shape->items.size() > (size_t)G4S_MAX_DIMS)
                    return store_fail(nullptr, G4S_ERR_UNSUPPORTED,
                                      "tensor %s has %zu dimensions (at most %d)", name.c_str(),
                                      shape->items.size(), G4S_MAX_DIMS);
                info.ndim = (int32_t)shape->items.size();
                for (int32_t d = 0; d < info.ndim; ++d) info.shape[d] = as_i32(&shape->items[d]);
            }
            st->tensor_lookup[name] = st->names.size(); /* AddOrSetValue */
            st->names.push_back(name);
            st->infos.push_back(info);
        }
    }
    if (st->infos.empty())
        return store_fail(nullptr, G4S_ERR_FORMAT, "Manifest lists no tensors");
    return G4S_OK;
}

int64_t q4_device_bytes(int32_t rows, int32_t cols, int32_t layout)
{
    if (rows < 1 || cols < 32 || cols % 32 != 0) return -1;
    const int64_t nblk = cols / 32;
    if (layout == G4S_Q4_LAYOUT_ROWS) return (int64_t)rows * nblk * 18;
    if (layout == G4S_Q4_LAYOUT_TILED64)
        return (int64_t)((rows + 63) / 64) * nblk * g4s::kQ4TileBytes;
    return -1;
}

}  // namespace

G4S_API int g4s_store_open(g4s_store** out, const char* vpk_path, const char* manifest_path,
                           const char* weights_path)
{
    g_open_error.clear();
    if (!out || !vpk_path) return store_fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "out or vpk_path is NULL");
    *out = nullptr;
    const char* mpath = manifest_path ? manifest_path : "E4B/manifest.json"; /* Types.pas:79 */
    const char* wpath = weights_path ? weights_path : "E4B/weights.bin";     /* Types.pas:85 */
    auto* st = new (std::nothrow) g4s_store();
    if (!st) return store_fail(nullptr, G4S_ERR_OUT_OF_MEMORY, "out of host memory");
    const std::string file = vpk_filename(vpk_path);
    int rc = vfs_open(st, file);
    if (rc == G4S_OK) {
        const Entry* me = find_entry(st, mpath);
        const uint8_t* mp = nullptr;
        if (!me)
            rc = store_fail(nullptr, G4S_ERR_NOT_FOUND, "Manifest not found in VPK: %s", mpath);
        else if ((rc = entry_view(st, *me, &mp, nullptr)) == G4S_OK)
            rc = parse_manifest(st, mp, me->size);
    }
    if (rc == G4S_OK) {
        const Entry* we = find_entry(st, wpath);
        const uint8_t* wp = nullptr;
        if (!we)
            rc = store_fail(nullptr, G4S_ERR_NOT_FOUND, "Weights file not found in VPK: %s", wpath);
        else if ((rc = entry_view(st, *we, &wp, nullptr)) == G4S_OK)
            st->weights_entry = (size_t)(we - st->entries.data());
    }
    if (rc != G4S_OK) {
        store_release(st);
        delete st;
        return rc;
    }
    *out = st;
    return G4S_OK;
}

G4S_API int g4s_store_close(g4s_store* st)
{
    if (!st) return G4S_OK;
    store_release(st);
    delete st;
    return G4S_OK;
}

G4S_API const char* g4s_store_last_error(const g4s_store* st)
{
    return st ? st->err.c_str() : g_open_error.c_str();
}

G4S_API int32_t g4s_store_tensor_count(const g4s_store* st)
{
    return st ? (int32_t)st->infos.size() : 0;
}

G4S_API int g4s_store_tensor_info(g4s_store* st, int32_t index, g4s_tensor_info* info,
                                  char* name, int32_t name_capacity)
{
    if (!st) return store_fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "store is NULL");
    if (index < 0 || (size_t)index >= st->infos.size())
        return store_fail(st, G4S_ERR_INVALID_ARGUMENT, "tensor index %d outside [0, %zu)", index,
                          st->infos.size());
    if (info) *info = st->infos[(size_t)index];
    if (name && name_capacity > 0) {
        const std::string& n = st->names[(size_t)index];
        if ((size_t)name_capacity <= n.size())
            return store_fail(st, G4S_ERR_INVALID_ARGUMENT, "name of tensor %d needs %zu bytes",
                              index, n.size() + 1);
        std::memcpy(name, n.c_str(), n.size() + 1);
    }
    return G4S_OK;
}

G4S_API int g4s_store_find_tensor(g4s_store* st, const char* name, g4s_tensor_info* info)
{
    if (!st || !name) return store_fail(st, G4S_ERR_INVALID_ARGUMENT, "store or name is NULL");
    const auto it = st->tensor_lookup.find(name);
    if (it == st->tensor_lookup.end()) {
        if (info) *info = g4s_tensor_info{};
        return store_fail(st, G4S_ERR_NOT_FOUND, "Tensor not found: %s", name);
    }
    if (info) *info = st->infos[it->second];
    return G4S_OK;
}

G4S_API const void* g4s_store_raw_pointer(g4s_store* st, const char* name)
{
    g4s_tensor_info info;
    if (g4s_store_find_tensor(st, name, &info) != G4S_OK) return nullptr;
    const Entry& we = st->entries[st->weights_entry];
    if (info.offset > we.size || info.size > we.size - info.offset) {
        store_fail(st, G4S_ERR_FORMAT, "tensor %s [%llu, +%llu) lies beyond the weights entry",
                   name, (unsigned long long)info.offset, (unsigned long long)info.size);
        return nullptr;
    }
    return st->base + we.offset + info.offset;
}

G4S_API int g4s_store_verify(g4s_store* st)
{
    if (!st) return store_fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "store is NULL");
    for (const Entry& en : st->entries) {
        const uint8_t* p = nullptr;
        const int rc = entry_view(st, en, &p, st);
        if (rc != G4S_OK) return rc;
        const uint32_t c = crc32_bytes(p, en.size);
        if (c != en.crc)
            return store_fail(st, G4S_ERR_FORMAT, "CRC-32 of %s is %08x, the directory says %08x",
                              en.path.c_str(), c, en.crc);
    }
    return G4S_OK;
}

G4S_API int64_t g4s_q4_0_device_bytes(int32_t rows, int32_t cols, int32_t layout)
{
    return q4_device_bytes(rows, cols, layout);
}

G4S_API int g4s_q4_0_repack(const void* d_rows, int32_t rows, int32_t cols, void* d_tiled,
                            void* hip_stream)
{
    g4s::clear_null_handle_error();
    if (!d_rows || !d_tiled)
        return g4s::set_null_handle_error(G4S_ERR_INVALID_ARGUMENT, "d_rows or d_tiled is NULL");
    if (q4_device_bytes(rows, cols, G4S_Q4_LAYOUT_ROWS) < 0)
        return g4s::set_null_handle_error(G4S_ERR_INVALID_ARGUMENT,
                                          "rows %d / cols %d: need rows >= 1, cols a multiple of 32",
                                          rows, cols);
    if ((reinterpret_cast<uintptr_t>(d_tiled) & 15u) != 0 || (reinterpret_cast<uintptr_t>(d_rows) & 1u) != 0)
        return g4s::set_null_handle_error(G4S_ERR_INVALID_ARGUMENT,
                                          "d_tiled must be 16-byte and d_rows 2-byte aligned");
    const hipError_t e = g4s::q4_tile_launch(static_cast<const uint8_t*>(d_rows), rows, cols / 32,
                                             static_cast<uint8_t*>(d_tiled),
                                             static_cast<hipStream_t>(hip_stream));
    if (e != hipSuccess)
        return g4s::set_null_handle_error(G4S_ERR_HIP, "repack launch: %s", hipGetErrorString(e));
    return G4S_OK;
}

/* TWeightStore.LoadTensor for a Q4_0 tensor (src/Gemma4.Tensors.pas:477-506)
 * and the engine's staged upload of it (src/Gemma4.Model.pas:494-640), into
 * the caller's device buffer in one of the sampler's layouts. */
G4S_API int g4s_store_upload_q4_0(g4s_store* st, const char* name, int32_t layout, void* d_dst,
                                  uint64_t dst_bytes, void* hip_stream)
{
    if (!st) return store_fail(nullptr, G4S_ERR_INVALID_ARGUMENT, "store is NULL");
    if (!name || !d_dst) return store_fail(st, G4S_ERR_INVALID_ARGUMENT, "name or d_dst is NULL");
    g4s_tensor_info info;
    int rc = g4s_store_find_tensor(st, name, &info);
    if (rc != G4S_OK) return rc;
    if (info.output_dtype != G4S_WDTYPE_Q4_0)
        return store_fail(st, G4S_ERR_UNSUPPORTED, "tensor %s is not Q4_0 (output dtype %d)", name,
                          info.output_dtype);
    if (info.ndim != 2 || info.shape[0] < 1 || info.shape[1] < 32 || info.shape[1] % 32 != 0)
        return store_fail(st, G4S_ERR_UNSUPPORTED,
                          "tensor %s: a Q4_0 matrix [rows, cols] with cols a multiple of 32 is "
                          "needed (ndim %d)", name, info.ndim);
    const int32_t rows = info.shape[0], cols = info.shape[1];
    const uint64_t want = (uint64_t)rows * (uint64_t)(cols / 32) * 18u;
    if (info.size != want)
        return store_fail(st, G4S_ERR_FORMAT,
                          "tensor %s: %llu bytes, a [%d, %d] Q4_0 matrix has %llu", name,
                          (unsigned long long)info.size, rows, cols, (unsigned long long)want);
    const int64_t need = q4_device_bytes(rows, cols, layout);
    if (need < 0) return store_fail(st, G4S_ERR_INVALID_ARGUMENT, "layout %d is unknown", layout);
    if (dst_bytes < (uint64_t)need)
        return store_fail(st, G4S_ERR_INVALID_ARGUMENT, "d_dst holds %llu bytes, the layout needs %lld",
                          (unsigned long long)dst_bytes, (long long)need);
    if ((reinterpret_cast<uintptr_t>(d_dst) & 15u) != 0)
        return store_fail(st, G4S_ERR_INVALID_ARGUMENT, "d_dst is not 16-byte aligned");
    const uint8_t* src = static_cast<const uint8_t*>(g4s_store_raw_pointer(st, name));
    if (!src) return G4S_ERR_FORMAT;

    /* Staged copies of whole 64-row groups through two pinned buffers; a
     * tiled upload lands each piece in a device staging buffer and repacks
     * it from there. */
    const hipStream_t s = static_cast<hipStream_t>(hip_stream);
    const uint64_t row_bytes = (uint64_t)(cols / 32) * 18u;
    const uint64_t group_bytes = 64u * row_bytes;
    uint64_t piece_rows = ((uint64_t)(16u << 20) / group_bytes) * 64u;
    if (piece_rows == 0) piece_rows = 64;
    const uint64_t piece_bytes = piece_rows * row_bytes;
    uint8_t* pin[2] = {nullptr, nullptr};
    uint8_t* dstage[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool recorded[2] = {false, false};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        e = hipHostMalloc(reinterpret_cast<void**>(&pin[i]), piece_bytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
        if (e == hipSuccess && layout == G4S_Q4_LAYOUT_TILED64)
            e = hipMalloc(reinterpret_cast<void**>(&dstage[i]), piece_bytes);
    }
    const char* what = "staging allocation";
    int slot = 0;
    for (uint64_t r0 = 0; e == hipSuccess && r0 < (uint64_t)rows; r0 += piece_rows, slot ^= 1) {
        const uint64_t nr = (uint64_t)rows - r0 < piece_rows ? (uint64_t)rows - r0 : piece_rows;
        const uint64_t nbytes = nr * row_bytes;
        if (recorded[slot]) {
            what = "staging wait";
            e = hipEventSynchronize(ev[slot]); /* the copy that last read this buffer is done */
            if (e != hipSuccess) break;
        }
        std::memcpy(pin[slot], src + r0 * row_bytes, nbytes);
        if (layout == G4S_Q4_LAYOUT_ROWS) {
            what = "weights copy";
            e = hipMemcpyAsync(static_cast<uint8_t*>(d_dst) + r0 * row_bytes, pin[slot], nbytes,
                               hipMemcpyHostToDevice, s);
        } else {
            what = "weights copy";
            e = hipMemcpyAsync(dstage[slot], pin[slot], nbytes, hipMemcpyHostToDevice, s);
            if (e == hipSuccess) {
                what = "repack launch";
                e = g4s::q4_tile_launch(dstage[slot], (int32_t)nr, cols / 32,
                                        static_cast<uint8_t*>(d_dst) +
                                            (r0 / 64) * (uint64_t)(cols / 32) * g4s::kQ4TileBytes,
                                        s);
            }
        }
        if (e == hipSuccess) {
            what = "event record";
            e = hipEventRecord(ev[slot], s);
            recorded[slot] = e == hipSuccess;
        }
    }
    if (e == hipSuccess) {
        what = "stream synchronize";
        e = hipStreamSynchronize(s);
    } else {
        /* copies and repacks enqueued before the failure may still read the
         * staging buffers freed below */
        (void)hipStreamSynchronize(s);
    }
    for (int i = 0; i < 2; ++i) {
        if (ev[i]) (void)hipEventDestroy(ev[i]);
        if (pin[i]) (void)hipHostFree(pin[i]);
        if (dstage[i]) (void)hipFree(dstage[i]);
    }
    if (e != hipSuccess)
        return store_fail(st, G4S_ERR_HIP, "upload of %s: %s: %s", name, what, hipGetErrorString(e));
    return G4S_OK;
}
