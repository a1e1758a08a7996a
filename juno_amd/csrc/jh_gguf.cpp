// jh_gguf.cpp -- GGUF reader and file -> HBM loader behind the C ABI.
//
// Restates GgufReader.open / meta* / tensor* / tensorRaw
// (/root/reference/node/src/main/java/cab/ml/juno/node/GgufReader.java:102-360)
// and the llamafile locator (findGgufOffsetInZip / findGgufOffsetByForwardScan
// / readZip64ExtraLocalOffset, :808-1154):
//
//  * header: magic "GGUF", version 2 or 3, tensor count, metadata count;
//  * metadata values are kept with the reference's Java typing: UINT8 / INT8
//    and UINT16 / INT16 read as sign-extended int, UINT32 / INT32 as int,
//    UINT64 / INT64 as long, FLOAT32 as float, FLOAT64 as double, BOOL,
//    STRING, ARRAY (the metaInt / metaLong / metaFloat getters follow
//    Number.intValue / longValue / floatValue);
//  * the data section starts at the next multiple of 32 bytes after the
//    tensor infos, relative to the start of the GGUF image (the reference's
//    fixed ALIGNMENT, :51, :168-176);
//  * a file that does not start with the magic is taken to be a llamafile (a
//    ZIP with the GGUF stored uncompressed): the end-of-central-directory
//    record is searched in the last 64 KiB + 22 bytes (ZIP64 resolved), else
//    a forward scan finds the first stored local entry named *.gguf.
//
// jh_gguf_upload streams one tensor from the file through pinned host staging
// into a device matrix (jh_qmat), with no intermediate copy of the whole
// tensor on the host and no 2 GiB byte[] limit.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <algorithm>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/junohip.h"

// jh_api.cpp: records msg as the thread's jh_last_error() (cleared for JH_OK) and returns code
extern "C" int jh_internal_fail(int code, const char *msg);

namespace {

int gfail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return jh_internal_fail(code, buf);
}

enum VType {
    V_UINT8 = 0, V_INT8 = 1, V_UINT16 = 2, V_INT16 = 3, V_UINT32 = 4, V_INT32 = 5, V_FLOAT32 = 6,
    V_BOOL = 7, V_STRING = 8, V_ARRAY = 9, V_UINT64 = 10, V_INT64 = 11, V_FLOAT64 = 12,
};

struct MetaValue {
    int vtype = -1;
    int64_t i = 0;      // integer kinds (Java int / long value)
    double f = 0;       // FLOAT32 (exact float value) / FLOAT64
    bool b = false;
    std::string s;
    int elem_type = -1;   // ARRAY
    int64_t count = 0;    // ARRAY
};

struct TensorInfo {
    std::string name;
    std::vector<int64_t> dims;
    int type = 0;
    int64_t offset = 0;  // relative to the data section
    int64_t nelems = 1;
};

}  // namespace

struct jh_gguf {
    int fd = -1;
    int64_t file_size = 0;
    int version = 0;
    int64_t gguf_offset = 0, data_offset = 0, metadata_end = 0, kv_count = 0;
    std::unordered_map<std::string, MetaValue> meta;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, int64_t> index;
};

namespace {

// Java long arithmetic (the reference's offsets and sizes are longs): products
// and sums wrap in two's complement instead of overflowing (undefined in C++);
// a wrapped value then fails the reads' bounds checks.
inline int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }
inline int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }

// ------------------------------------------------------------------ positional reads
struct Reader {
    int fd;
    int64_t size;
    bool ok = true;
    bool read(int64_t pos, void *dst, size_t n) {
        if (!ok || pos < 0 || pos > size || n > (uint64_t)(size - pos)) return ok = false;
        uint8_t *p = static_cast<uint8_t *>(dst);
        while (n) {
            const ssize_t r = pread(fd, p, n, pos);
            if (r <= 0) return ok = false;
            p += r;
            pos += r;
            n -= (size_t)r;
        }
        return true;
    }
    template <typename T> T get(int64_t &pos) {
        T v{};
        if (read(pos, &v, sizeof v)) pos += sizeof v;
        return v;
    }
    std::string str(int64_t &pos) {  // readString: uint64 length + UTF-8 bytes
        const uint64_t len = get<uint64_t>(pos);
        if (!ok || len > (uint64_t)(size - pos)) {
            ok = false;
            return {};
        }
        std::string s((size_t)len, '\0');
        if (len && read(pos, &s[0], (size_t)len)) pos += (int64_t)len;
        return s;
    }
};

// readMetadataValue / readArray (:1189-1246) with Java's typing; arrays are skipped past
// and summarised (element type, count), which is all the reader's users need.
bool read_value(Reader &rd, int64_t &pos, int vtype, MetaValue *out, int depth) {
    MetaValue v;
    v.vtype = vtype;
    switch (vtype) {
    case V_UINT8:
    case V_INT8: v.i = (int8_t)rd.get<uint8_t>(pos); break;
    case V_UINT16:
    case V_INT16: v.i = (int16_t)rd.get<uint16_t>(pos); break;
    case V_UINT32:
    case V_INT32: v.i = (int32_t)rd.get<uint32_t>(pos); break;
    case V_FLOAT32: {
        const float f = rd.get<float>(pos);
        v.f = f;
        break;
    }
    case V_BOOL: v.b = rd.get<uint8_t>(pos) != 0; break;
    case V_STRING: v.s = rd.str(pos); break;
    case V_UINT64:
    case V_INT64: v.i = (int64_t)rd.get<uint64_t>(pos); break;
    case V_FLOAT64: v.f = rd.get<double>(pos); break;
    case V_ARRAY: {
        if (depth > 4) return false;
        v.elem_type = (int32_t)rd.get<uint32_t>(pos);
        v.count = (int64_t)rd.get<uint64_t>(pos);
        if (v.count < 0) return false;
        for (int64_t k = 0; k < v.count && rd.ok; k++)
            if (!read_value(rd, pos, v.elem_type, nullptr, depth + 1)) return false;
        break;
    }
    default: return false;
    }
    if (out) *out = std::move(v);
    return rd.ok;
}

// ------------------------------------------------------------------ llamafile (ZIP) locator
int64_t rd_u32(const uint8_t *p) { return (int64_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24)); }
int rd_u16(const uint8_t *p) { return p[0] | (p[1] << 8); }
int64_t rd_u64(const uint8_t *p) { return (int64_t)((uint64_t)rd_u32(p) | ((uint64_t)rd_u32(p + 4) << 32)); }
bool ends_with_gguf(const std::string &s) { return s.size() >= 5 && s.compare(s.size() - 5, 5, ".gguf") == 0; }

// findGgufOffsetByForwardScan (:1027-1134): first STORED local entry *.gguf
int64_t forward_scan(Reader &rd) {
    const int64_t n = rd.size;
    std::vector<uint8_t> buf(1 << 20);
    for (int64_t base = 0; base + 4 <= n; base += (int64_t)buf.size() - 3) {
        const size_t len = (size_t)std::min<int64_t>((int64_t)buf.size(), n - base);
        if (!rd.read(base, buf.data(), len)) return -1;
        for (size_t i = 0; i + 4 <= len; i++) {
            if (rd_u32(&buf[i]) != 0x04034b50) continue;
            const int64_t abs = base + (int64_t)i;
            uint8_t lh[30];
            if (abs + 30 > n || !rd.read(abs, lh, 30)) {
                rd.ok = true;
                continue;
            }
            if (rd_u16(lh + 8) != 0) continue;  // compression: STORED only
            const int fn = rd_u16(lh + 26), ex = rd_u16(lh + 28);
            if (fn == 0 || fn > 512 || abs + 30 + fn > n) continue;
            std::string name((size_t)fn, '\0');
            if (!rd.read(abs + 30, &name[0], (size_t)fn)) return -1;
            if (ends_with_gguf(name)) return abs + 30 + fn + ex;
        }
        if ((int64_t)len < (int64_t)buf.size()) break;
    }
    return -1;
}

// findGgufOffsetInZip (:808-1025)
int64_t zip_offset(Reader &rd, std::string *why) {
    const int64_t n = rd.size;
    const int64_t search = std::min<int64_t>(n, 65535 + 22), start = n - search;
    std::vector<uint8_t> tail((size_t)search);
    if (!rd.read(start, tail.data(), tail.size())) return -1;
    int64_t eocd = -1;
    for (int64_t i = search - 22; i >= 0; i--) {
        if (rd_u32(&tail[i]) != 0x06054b50) continue;
        const int64_t cd_size = rd_u32(&tail[i + 12]), cd_off = rd_u32(&tail[i + 16]), at = start + i;
        const bool z64 = cd_size == 0xFFFFFFFFLL || cd_off == 0xFFFFFFFFLL;
        if (!z64 && (cd_size == 0 || cd_size > at || cd_off + cd_size > at || cd_off >= n)) continue;
        eocd = i;
        break;
    }
    if (eocd < 0) return forward_scan(rd);
    int64_t cd_size = rd_u32(&tail[eocd + 12]), cd_off = rd_u32(&tail[eocd + 16]);
    if (cd_size == 0xFFFFFFFFLL || cd_off == 0xFFFFFFFFLL) {  // ZIP64 locator right before the EOCD
        const int64_t loc = start + eocd - 20;
        uint8_t l[20], z[56];
        if (loc < 0 || !rd.read(loc, l, 20) || rd_u32(l) != 0x07064b50) {
            *why = "ZIP64 EOCD locator signature not found";
            return -1;
        }
        const int64_t zpos = rd_u64(l + 8);
        if (!rd.read(zpos, z, 56) || rd_u32(z) != 0x06064b50) {
            *why = "ZIP64 EOCD record signature not found";
            return -1;
        }
        cd_size = rd_u64(z + 40);
        cd_off = rd_u64(z + 48);
    }
    if (cd_size == 0) {
        *why = "ZIP central directory is empty - no entries in llamafile";
        return -1;
    }
    if (cd_off >= n) {
        *why = "ZIP CD offset is beyond the file size";
        return -1;
    }
    if (cd_size > n - cd_off) cd_size = n - cd_off;  // a truncated directory is parsed as far as it goes
    std::vector<uint8_t> cd((size_t)cd_size);
    if (!rd.read(cd_off, cd.data(), cd.size())) return -1;
    for (size_t p = 0; p + 46 <= cd.size();) {
        if (rd_u32(&cd[p]) != 0x02014b50) break;
        const int fn = rd_u16(&cd[p + 28]), ex = rd_u16(&cd[p + 30]), cm = rd_u16(&cd[p + 32]);
        int64_t lho = rd_u32(&cd[p + 42]);
        const size_t next = p + 46 + fn + ex + cm;
        if (next > cd.size()) break;
        const std::string name(reinterpret_cast<const char *>(&cd[p + 46]), (size_t)fn);
        if (ends_with_gguf(name)) {
            if (lho == 0xFFFFFFFFLL) {  // readZip64ExtraLocalOffset (:1136-1154)
                bool found = false;
                for (size_t e = p + 46 + fn; e + 4 <= p + 46 + fn + ex;) {
                    const int id = rd_u16(&cd[e]), sz = rd_u16(&cd[e + 2]);
                    if (id == 0x0001 && e + 4 + 16 + 8 <= p + 46 + fn + ex) {
                        lho = rd_u64(&cd[e + 4 + 16]);
                        found = true;
                        break;
                    }
                    e += 4 + (size_t)sz;
                }
                if (!found) {
                    *why = "ZIP64 extra field with local-header offset not found";
                    return -1;
                }
            }
            uint8_t lh[30];
            if (!rd.read(lho, lh, 30) || rd_u32(lh) != 0x04034b50) {
                *why = "bad local file header signature";
                return -1;
            }
            return lho + 30 + rd_u16(lh + 26) + rd_u16(lh + 28);
        }
        p = next;
    }
    *why = "No .gguf entry found in the ZIP central directory of this llamafile";
    return -1;
}

constexpr uint32_t kMagic = 0x46554747;  // "GGUF"
constexpr int64_t kAlign = 32;

bool raw_bytes(int type, int64_t nelems, int64_t *out) {  // rawByteCount (:347-360)
    switch (type) {
    case 0: *out = wmul(nelems, 4); return true;
    case 1:
    case 30: *out = wmul(nelems, 2); return true;
    case 8: *out = wmul(nelems / 32, 34); return true;
    case 2: *out = wmul(nelems / 32, 18); return true;
    case 10: *out = wmul(nelems / 256, 84); return true;
    case 11: *out = wmul(nelems / 256, 110); return true;
    case 12: *out = wmul(nelems / 256, 144); return true;
    case 13: *out = wmul(nelems / 256, 176); return true;
    case 14: *out = wmul(nelems / 256, 210); return true;
    default: return false;
    }
}

const MetaValue *find_meta(const jh_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

bool is_number(const MetaValue &v) {
    switch (v.vtype) {
    case V_UINT8: case V_INT8: case V_UINT16: case V_INT16: case V_UINT32: case V_INT32:
    case V_UINT64: case V_INT64: case V_FLOAT32: case V_FLOAT64: return true;
    default: return false;
    }
}
bool is_float(int t) { return t == V_FLOAT32 || t == V_FLOAT64; }

}  // namespace

extern "C" {

int jh_gguf_open(const char *path, jh_gguf **out) {
    if (!path || !out) return gfail(JH_EINVAL, "path and out must not be null");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return gfail(JH_EIO, "cannot open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return gfail(JH_EIO, "cannot stat %s: %s", path, strerror(errno));
    }
    jh_gguf *g = new jh_gguf;
    g->fd = fd;
    g->file_size = st.st_size;
    Reader rd{fd, (int64_t)st.st_size};
    auto bad = [&](int code, const char *fmt, auto... a) {
        jh_gguf_close(g);
        return gfail(code, fmt, a...);
    };
    uint32_t magic = 0;
    if (!rd.read(0, &magic, 4)) return bad(JH_EFORMAT, "Not a GGUF file (shorter than 4 bytes)");
    if (magic != kMagic) {
        std::string why;
        const int64_t off = zip_offset(rd, &why);
        rd.ok = true;
        if (off < 0)
            return bad(JH_EFORMAT, "%s", why.empty() ? "No valid ZIP EOCD record found - file is neither a GGUF nor a llamafile ZIP"
                                                     : why.c_str());
        g->gguf_offset = off;
    }
    int64_t pos = g->gguf_offset;
    magic = rd.get<uint32_t>(pos);
    const int32_t version = (int32_t)rd.get<uint32_t>(pos);
    const int64_t n_tensors = (int64_t)rd.get<uint64_t>(pos), n_kv = (int64_t)rd.get<uint64_t>(pos);
    if (!rd.ok || magic != kMagic)
        return bad(JH_EFORMAT, "Not a GGUF file (magic=0x%x at offset %lld)", magic, (long long)g->gguf_offset);
    if (version < 2 || version > 3) return bad(JH_EFORMAT, "Unsupported GGUF version: %d", version);
    if (n_tensors < 0 || n_kv < 0 || n_tensors > (1 << 24) || n_kv > (1 << 24))
        return bad(JH_EFORMAT, "implausible GGUF counts: tensors=%lld metadata=%lld", (long long)n_tensors,
                   (long long)n_kv);
    g->version = version;
    g->kv_count = n_kv;
    for (int64_t i = 0; i < n_kv; i++) {
        std::string key = rd.str(pos);
        const int vtype = (int32_t)rd.get<uint32_t>(pos);
        MetaValue v;
        if (!rd.ok || !read_value(rd, pos, vtype, &v, 0))
            return bad(JH_EFORMAT, "bad metadata entry %lld (type %d)", (long long)i, vtype);
        g->meta[std::move(key)] = std::move(v);  // a repeated key keeps the last value, like HashMap.put
    }
    g->metadata_end = pos;
    for (int64_t i = 0; i < n_tensors; i++) {
        TensorInfo t;
        t.name = rd.str(pos);
        const int32_t nd = (int32_t)rd.get<uint32_t>(pos);
        if (!rd.ok || nd < 0 || nd > 8) return bad(JH_EFORMAT, "bad tensor info %lld", (long long)i);
        for (int d = 0; d < nd; d++) {
            const int64_t v = (int64_t)rd.get<uint64_t>(pos);
            t.dims.push_back(v);
            t.nelems = wmul(t.nelems, v);  // :162-164
        }
        t.type = (int32_t)rd.get<uint32_t>(pos);
        t.offset = (int64_t)rd.get<uint64_t>(pos);
        if (!rd.ok) return bad(JH_EFORMAT, "truncated tensor info %lld", (long long)i);
        g->index[t.name] = (int64_t)g->tensors.size();
        g->tensors.push_back(std::move(t));
    }
    const int64_t rel = pos - g->gguf_offset;
    g->data_offset = g->gguf_offset + (rel + kAlign - 1) / kAlign * kAlign;
    *out = g;
    return jh_internal_fail(JH_OK, "");
}

int jh_gguf_close(jh_gguf *g) {
    if (!g) return JH_OK;
    if (g->fd >= 0) ::close(g->fd);
    delete g;
    return JH_OK;
}

int jh_gguf_info(const jh_gguf *g, int *version, int64_t *tensor_count, int64_t *kv_count, int64_t *gguf_offset,
                 int64_t *data_offset, int64_t *metadata_end) {
    if (!g) return gfail(JH_EINVAL, "gguf handle must not be null");
    if (version) *version = g->version;
    if (tensor_count) *tensor_count = (int64_t)g->tensors.size();
    if (kv_count) *kv_count = g->kv_count;
    if (gguf_offset) *gguf_offset = g->gguf_offset;
    if (data_offset) *data_offset = g->data_offset;
    if (metadata_end) *metadata_end = g->metadata_end;
    return JH_OK;
}

int jh_gguf_meta_type(const jh_gguf *g, const char *key, int *vtype, int *elem_type, int64_t *count) {
    if (!g || !key || !vtype) return gfail(JH_EINVAL, "gguf, key and vtype must not be null");
    const MetaValue *v = find_meta(g, key);
    *vtype = v ? v->vtype : -1;
    if (elem_type) *elem_type = v ? v->elem_type : -1;
    if (count) *count = v && v->vtype == V_ARRAY ? v->count : 0;
    return JH_OK;
}

int jh_gguf_meta_number(const jh_gguf *g, const char *key, int *present, int64_t *as_long, double *as_double) {
    if (!g || !key || !present) return gfail(JH_EINVAL, "gguf, key and present must not be null");
    const MetaValue *v = find_meta(g, key);
    *present = v && is_number(*v);
    if (!*present) return JH_OK;
    if (is_float(v->vtype)) {
        if (as_double) *as_double = v->f;
        if (as_long) {  // Number.longValue of a Float / Double: truncation, NaN -> 0, saturating
            const double f = v->f;
            *as_long = f != f ? 0 : f >= 9.2233720368547758e18 ? INT64_MAX : f <= -9.2233720368547758e18 ? INT64_MIN : (int64_t)f;
        }
    } else {
        if (as_long) *as_long = v->i;
        if (as_double) *as_double = (double)v->i;
    }
    return JH_OK;
}

int jh_gguf_meta_bool(const jh_gguf *g, const char *key, int *present, int *value) {
    if (!g || !key || !present || !value) return gfail(JH_EINVAL, "gguf, key, present and value must not be null");
    const MetaValue *v = find_meta(g, key);
    *present = v && v->vtype == V_BOOL;
    *value = *present && v->b;
    return JH_OK;
}

int jh_gguf_meta_string(const jh_gguf *g, const char *key, char *buf, size_t cap, size_t *len) {
    if (!g || !key || !len) return gfail(JH_EINVAL, "gguf, key and len must not be null");
    const MetaValue *v = find_meta(g, key);
    if (!v || v->vtype != V_STRING) {
        *len = (size_t)-1;  // absent or not a String (metaString returns null)
        return JH_OK;
    }
    *len = v->s.size();
    if (buf && cap) {
        const size_t n = std::min(cap - 1, v->s.size());
        memcpy(buf, v->s.data(), n);
        buf[n] = '\0';
    }
    return JH_OK;
}

int jh_gguf_tensor_index(const jh_gguf *g, const char *name, int64_t *index) {
    if (!g || !name || !index) return gfail(JH_EINVAL, "gguf, name and index must not be null");
    auto it = g->index.find(name);
    *index = it == g->index.end() ? -1 : it->second;
    return JH_OK;
}

int jh_gguf_tensor_info(const jh_gguf *g, int64_t index, const char **name, int *type, int *ndims, int64_t dims[8],
                        int64_t *nelems, int64_t *abs_offset) {
    if (!g) return gfail(JH_EINVAL, "gguf handle must not be null");
    if (index < 0 || index >= (int64_t)g->tensors.size())
        return gfail(JH_EINVAL, "Tensor index %lld out of range (available: %zu tensors)", (long long)index,
                     g->tensors.size());
    const TensorInfo &t = g->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (ndims) *ndims = (int)t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size(); d++) dims[d] = t.dims[d];
    if (nelems) *nelems = t.nelems;
    if (abs_offset) *abs_offset = wadd(g->data_offset, t.offset);
    return JH_OK;
}

int jh_gguf_tensor_read(const jh_gguf *g, int64_t index, void *dst, size_t cap, size_t *nbytes) {
    if (!g) return gfail(JH_EINVAL, "gguf handle must not be null");
    if (!dst && cap) return gfail(JH_EINVAL, "dst must not be null");
    if (index < 0 || index >= (int64_t)g->tensors.size())
        return gfail(JH_EINVAL, "Tensor index %lld out of range", (long long)index);
    const TensorInfo &t = g->tensors[(size_t)index];
    int64_t n = 0;
    if (!raw_bytes(t.type, t.nelems, &n)) return gfail(JH_EUNSUPPORTED, "No byte-size formula for GGML type %d", t.type);
    if (nbytes) *nbytes = (size_t)n;
    if (!dst) return JH_OK;  // size query
    if ((size_t)n > cap) return gfail(JH_EINVAL, "buffer of %zu bytes is smaller than the tensor (%lld bytes)", cap, (long long)n);
    Reader rd{g->fd, g->file_size};
    if (n < 0 || !rd.read(wadd(g->data_offset, t.offset), dst, (size_t)n))
        return gfail(JH_EIO, "Expected %lld bytes of %s at offset %lld", (long long)n, t.name.c_str(),
                     (long long)wadd(g->data_offset, t.offset));
    return JH_OK;
}

}  // extern "C"

// jh_gguf_upload lives in jh_api.cpp (it needs the jh_qmat internals); this
// helper streams a tensor's bytes into device memory through pinned staging.
int jh_gguf_stream_to_device(const jh_gguf *g, int64_t index, uint8_t *d_dst, int64_t *nbytes_out, int *type_out,
                             int64_t *rows_out, int64_t *cols_out) {
    if (!g) return gfail(JH_EINVAL, "gguf handle must not be null");
    if (index < 0 || index >= (int64_t)g->tensors.size())
        return gfail(JH_EINVAL, "Tensor index %lld out of range", (long long)index);
    const TensorInfo &t = g->tensors[(size_t)index];
    int64_t n = 0;
    if (!raw_bytes(t.type, t.nelems, &n)) return gfail(JH_EUNSUPPORTED, "No byte-size formula for GGML type %d", t.type);
    if (n < 0 || t.nelems < 0 || (!t.dims.empty() && t.dims[0] <= 0))
        return gfail(JH_EFORMAT, "tensor %s: bad shape (nelems %lld, dims[0] %lld)", t.name.c_str(),
                     (long long)t.nelems, (long long)(t.dims.empty() ? 1 : t.dims[0]));
    if (nbytes_out) *nbytes_out = n;
    if (type_out) *type_out = t.type;
    if (cols_out) *cols_out = t.dims.empty() ? 1 : t.dims[0];
    if (rows_out) *rows_out = t.dims.empty() ? 1 : t.nelems / t.dims[0];
    if (!d_dst) return JH_OK;  // shape query
    constexpr size_t kChunk = 32u << 20;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = JH_OK;
    for (int k = 0; k < 2 && rc == JH_OK; k++) {
        if (hipHostMalloc(&stage[k], kChunk, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&done[k], hipEventDisableTiming) != hipSuccess)
            rc = gfail(JH_ENOMEM, "hipHostMalloc failed: %zu bytes of pinned staging", kChunk);
    }
    hipStream_t s = nullptr;
    if (rc == JH_OK && hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess)
        rc = gfail(JH_EHIP, "hipStreamCreate failed");
    Reader rd{g->fd, g->file_size};
    int64_t at = 0;
    for (int k = 0; rc == JH_OK && at < n; k ^= 1) {
        const size_t len = (size_t)std::min<int64_t>((int64_t)kChunk, n - at);
        if (hipEventSynchronize(done[k]) != hipSuccess) {  // the previous copy out of this buffer
            rc = gfail(JH_EHIP, "hipEventSynchronize failed");
            break;
        }
        if (!rd.read(wadd(wadd(g->data_offset, t.offset), at), stage[k], len)) {
            rc = gfail(JH_EIO, "Expected %lld bytes of %s at offset %lld", (long long)n, t.name.c_str(),
                       (long long)wadd(g->data_offset, t.offset));
            break;
        }
        if (hipMemcpyAsync(d_dst + at, stage[k], len, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipEventRecord(done[k], s) != hipSuccess) {
            rc = gfail(JH_EHIP, "hipMemcpyAsync(H2D) failed");
            break;
        }
        at += (int64_t)len;
    }
    if (s) {
        if (hipStreamSynchronize(s) != hipSuccess && rc == JH_OK) rc = gfail(JH_EHIP, "hipStreamSynchronize failed");
        (void)hipStreamDestroy(s);
    }
    for (int k = 0; k < 2; k++) {
        if (done[k]) (void)hipEventDestroy(done[k]);
        if (stage[k]) (void)hipHostFree(stage[k]);
    }
    return rc;
}
