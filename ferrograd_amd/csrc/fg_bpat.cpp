// fg_bpat.cpp -- bpat tensor files: save device (or host) tensors, parse a
// file into host memory, upload its tensors into device memory.  Plan
// checkpoints (parameters and optimiser state) are built on these in
// fg_graph.cpp.
//
// Formats (crates/fused_gpu/src/io/headers.rs:1-117, readers and writers in
// io/versions/v0_v2.rs:22-300 and v1.rs:24-289), all little-endian, after
// the magic a u8 tensor count, then per tensor its rank, dims and data:
//   V0       "bpat"        u64 rank, u64 dims, f64 data
//   V1       "BPATv1\0\0"  u64 rank, u64 dims, f64 data, u32 tensor CRC;
//                          then a u32 CRC of every preceding byte
//   V1M      "BPATv1m\0"   as V1 with u32 rank / dims and f32 data
//   V2 f16   "BPAT\0f16"   u32 rank, u32 dims, f16 data
//   V2 bf16  "BPATbf16"    u32 rank, u32 dims, bf16 data
//   V2 f32   "BPAT\0f32"   u32 rank, u32 dims, f32 data
// CRCs are CRC-32 (IEEE 802.3, reflected 0xEDB88320, as crc32fast); a
// tensor's CRC covers its rank, dims and data bytes, and the file CRC is the
// CRC of all bytes before it (what crc32fast's combine of the tensor hasher
// plus the update with the tensor CRC amounts to, v1.rs:59-146).
//
// Departures from the reference (each corrects a defect):
//  * V1M dims are written as u32, as headers.rs documents and the V1M
//    reader reads; the reference's writer emits u64 dims (v1.rs:91-99).
//  * V1 / V1M readers skip and verify each tensor CRC and the file CRC; the
//    reference's load_tensors_v1 reads the next tensor's rank from the CRC
//    bytes (v1.rs:154-207) and nothing is verified.
//  * Element types convert on save and on upload (fp32 <-> fp64 / fp16 /
//    bf16, rounding to nearest even when narrowing); the reference requires
//    the device tensor to already hold the file's element type.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "fg_internal.h"

namespace {

constexpr int kMaxRank = 8;

struct Format {
    const char *magic;
    int magic_len;
    int dim_bytes;   // rank and dims
    int elem;        // element kind: kE64, kE32, kE16, kEB16
    bool crc;
};

enum { kE64 = 0, kE32 = 1, kE16 = 2, kEB16 = 3 };

const Format kFormats[] = {
    {"bpat", 4, 8, kE64, false},           // FG_BPAT_V0
    {"BPATv1\0\0", 8, 8, kE64, true},      // FG_BPAT_V1
    {"BPATv1m\0", 8, 4, kE32, true},       // FG_BPAT_V1M
    {"BPAT\0f16", 8, 4, kE16, false},      // FG_BPAT_V2_F16
    {"BPATbf16", 8, 4, kEB16, false},      // FG_BPAT_V2_BF16
    {"BPAT\0f32", 8, 4, kE32, false},      // FG_BPAT_V2_F32
};
constexpr int kNumFormats = 6;

int elem_bytes(int e) { return e == kE64 ? 8 : e == kE32 ? 4 : 2; }

// ---------------------------------------------------------------- CRC-32
uint32_t crc_table_entry(uint32_t i) {
    uint32_t c = i;
    for (int k = 0; k < 8; ++k) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
    return c;
}
struct Crc {
    uint32_t t[256];
    Crc() {
        for (uint32_t i = 0; i < 256; ++i) t[i] = crc_table_entry(i);
    }
};
const Crc &crc_tab() {
    static const Crc c;
    return c;
}
// Running CRC state (pre- and post-conditioned by crc32_finish).
uint32_t crc32_update(uint32_t state, const void *data, size_t n) {
    const uint8_t *p = static_cast<const uint8_t *>(data);
    const Crc &c = crc_tab();
    for (size_t i = 0; i < n; ++i) state = c.t[(state ^ p[i]) & 0xFFu] ^ (state >> 8);
    return state;
}
constexpr uint32_t kCrcInit = 0xFFFFFFFFu;
uint32_t crc32_finish(uint32_t state) { return state ^ 0xFFFFFFFFu; }

// ------------------------------------------------- 16-bit conversions
uint16_t f32_to_f16_bits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to infinity
    if (a < 0x38800000u) {                                     // f16 subnormal or zero
        // a as a multiple of 2^-24, rounded to nearest even by the FPU.
        const float v = std::nearbyint(std::ldexp(std::fabs(x), 24));
        return (uint16_t)(sign | (uint32_t)v);
    }
    uint32_t q = ((a >> 23) - 112u) << 10 | ((a >> 13) & 0x3FFu);
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}
float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    float r;
    if (e == 0) {
        r = std::ldexp((float)m, -24);
        if (sign) r = -r;
        return r;
    }
    const uint32_t u = e == 31 ? sign | 0x7F800000u | (m << 13) : sign | ((e + 112u) << 23) | (m << 13);
    std::memcpy(&r, &u, 4);
    return r;
}
uint16_t f32_to_bf16_bits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
float bf16_bits_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

// Element of a file buffer (element kind e) as double, and back.
double file_get(const uint8_t *p, int e, uint64_t i) {
    switch (e) {
        case kE64: { double d; std::memcpy(&d, p + 8 * i, 8); return d; }
        case kE32: { float f; std::memcpy(&f, p + 4 * i, 4); return f; }
        case kE16: { uint16_t h; std::memcpy(&h, p + 2 * i, 2); return f16_bits_to_f32(h); }
        default: { uint16_t h; std::memcpy(&h, p + 2 * i, 2); return bf16_bits_to_f32(h); }
    }
}

// Device-side element types (FG_DTYPE_*) as element kinds.
int elem_of_dtype(int dt) { return dt == FG_DTYPE_F16 ? kE16 : dt == FG_DTYPE_BF16 ? kEB16 : kE32; }

// Convert n elements between element kinds (narrowing rounds to nearest
// even; f64 -> 16-bit goes through f32, exact for values f32 holds).
void convert(const uint8_t *src, int se, uint8_t *dst, int de, uint64_t n) {
    if (se == de) {
        std::memcpy(dst, src, n * elem_bytes(se));
        return;
    }
    for (uint64_t i = 0; i < n; ++i) {
        const double v = file_get(src, se, i);
        switch (de) {
            case kE64: std::memcpy(dst + 8 * i, &v, 8); break;
            case kE32: { const float f = (float)v; std::memcpy(dst + 4 * i, &f, 4); break; }
            case kE16: { const uint16_t h = f32_to_f16_bits((float)v); std::memcpy(dst + 2 * i, &h, 2); break; }
            default: { const uint16_t h = f32_to_bf16_bits((float)v); std::memcpy(dst + 2 * i, &h, 2); break; }
        }
    }
}

void put_le(std::vector<uint8_t> &out, uint64_t v, int bytes) {
    for (int k = 0; k < bytes; ++k) out.push_back((uint8_t)(v >> (8 * k)));
}

struct FileTensor {
    int rank = 0;
    uint32_t shape[kMaxRank] = {};
    uint64_t numel = 0;
    uint64_t offset = 0;  // of the data in the file image
};

}  // namespace

struct fg_bpat {
    int header = 0;
    std::vector<uint8_t> image;  // the whole file
    std::vector<FileTensor> tensors;
};

namespace {

int serial_err(const char *what, const std::string &path) {
    fg::set_error("bpat %s: %s", path.c_str(), what);
    return FG_ERR_SERIALIZATION;
}

// Parse a file image (validates the structure and, for V1 / V1M, the CRCs).
int parse(fg_bpat &f, const std::string &path) {
    const std::vector<uint8_t> &b = f.image;
    int hdr = -1;
    for (int k = 0; k < kNumFormats; ++k) {
        const Format &F = kFormats[k];
        if (b.size() >= (size_t)F.magic_len && std::memcmp(b.data(), F.magic, F.magic_len) == 0) {
            hdr = k;
            break;
        }
    }
    if (hdr < 0) return serial_err("invalid magic header", path);
    const Format &F = kFormats[hdr];
    f.header = hdr;
    uint64_t off = F.magic_len;
    if (off + 1 > b.size()) return serial_err("unexpected end of file (count)", path);
    const int count = b[off++];
    auto get = [&](int bytes, uint64_t &v) {
        if (off + bytes > b.size()) return false;
        v = 0;
        for (int k = 0; k < bytes; ++k) v |= (uint64_t)b[off + k] << (8 * k);
        off += bytes;
        return true;
    };
    for (int t = 0; t < count; ++t) {
        FileTensor ft;
        const uint64_t start = off;
        uint64_t rank;
        if (!get(F.dim_bytes, rank)) return serial_err("unexpected end of file (rank)", path);
        if (rank > kMaxRank) return serial_err("tensor rank above 8", path);
        ft.rank = (int)rank;
        ft.numel = 1;
        for (int d = 0; d < ft.rank; ++d) {
            uint64_t dim;
            if (!get(F.dim_bytes, dim)) return serial_err("unexpected end of file (dims)", path);
            if (dim > 0xFFFFFFFFull) return serial_err("dimension above u32", path);
            ft.shape[d] = (uint32_t)dim;
            ft.numel *= dim;
            if (ft.numel > (1ull << 40)) return serial_err("tensor too large", path);
        }
        ft.offset = off;
        const uint64_t nbytes = ft.numel * elem_bytes(F.elem);
        if (off + nbytes > b.size()) return serial_err("unexpected end of file (data)", path);
        off += nbytes;
        if (F.crc) {
            uint64_t stored;
            if (!get(4, stored)) return serial_err("unexpected end of file (tensor CRC)", path);
            const uint32_t c = crc32_finish(crc32_update(kCrcInit, b.data() + start, off - 4 - start));
            if (c != (uint32_t)stored) return serial_err("tensor checksum mismatch", path);
        }
        f.tensors.push_back(ft);
    }
    if (F.crc) {
        uint64_t stored;
        const uint64_t body = off;
        if (!get(4, stored)) return serial_err("unexpected end of file (file CRC)", path);
        if (crc32_finish(crc32_update(kCrcInit, b.data(), body)) != (uint32_t)stored)
            return serial_err("file checksum mismatch", path);
    }
    if (off != b.size()) return serial_err("trailing bytes after the last tensor", path);
    return FG_OK;
}

}  // namespace

namespace {

// Shared by the device and host savers: `fetch` copies a tensor's raw
// elements (its dtype) into the given buffer.
template <class Fetch>
int save_impl(const char *path, int header, int n, const fg_bpat_tensor *tensors, Fetch fetch,
              const char *who) {
    FG_REQUIRE(path && (tensors || n == 0), FG_ERR_INVALID_ARGUMENT, "%s: NULL argument", who);
    FG_REQUIRE(header >= 0 && header < kNumFormats, FG_ERR_INVALID_ARGUMENT,
               "%s: unknown header %d", who, header);
    FG_REQUIRE(n >= 0 && n <= 255, FG_ERR_INVALID_ARGUMENT,
               "%s: %d tensors (a file holds at most 255)", who, n);
    const Format &F = kFormats[header];
    std::vector<uint8_t> out(F.magic, F.magic + F.magic_len);
    out.push_back((uint8_t)n);
    std::vector<uint8_t> raw, conv;
    for (int t = 0; t < n; ++t) {
        const fg_bpat_tensor &T = tensors[t];
        FG_REQUIRE(T.rank >= 0 && T.rank <= kMaxRank, FG_ERR_INVALID_ARGUMENT,
                   "%s: tensor %d has rank %d", who, t, T.rank);
        FG_REQUIRE(T.dtype >= FG_DTYPE_F32 && T.dtype <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
                   "%s: tensor %d has unknown dtype %d", who, t, T.dtype);
        uint64_t numel = 1;
        for (int d = 0; d < T.rank; ++d) numel *= T.shape[d];
        FG_REQUIRE(numel == 0 || T.d_ptr, FG_ERR_INVALID_ARGUMENT, "%s: tensor %d has no data",
                   who, t);
        const uint64_t start = out.size();
        put_le(out, (uint64_t)T.rank, F.dim_bytes);
        for (int d = 0; d < T.rank; ++d) put_le(out, T.shape[d], F.dim_bytes);
        const int de = elem_of_dtype(T.dtype);
        raw.resize(numel * elem_bytes(de));
        if (numel) {
            const int rc = fetch(T, raw);
            if (rc) return rc;
        }
        conv.resize(numel * elem_bytes(F.elem));
        convert(raw.data(), de, conv.data(), F.elem, numel);
        out.insert(out.end(), conv.begin(), conv.end());
        if (F.crc) {
            const uint32_t c = crc32_finish(crc32_update(kCrcInit, out.data() + start,
                                                         out.size() - start));
            put_le(out, c, 4);
        }
    }
    if (F.crc) put_le(out, crc32_finish(crc32_update(kCrcInit, out.data(), out.size())), 4);
    FILE *fp = std::fopen(path, "wb");
    if (!fp) {
        fg::set_error("bpat %s: cannot open for writing", path);
        return FG_ERR_FILE_NOT_FOUND;
    }
    const bool ok = std::fwrite(out.data(), 1, out.size(), fp) == out.size();
    const bool closed = std::fclose(fp) == 0;
    if (!ok || !closed) return serial_err("write failed", path);
    return FG_OK;
}

}  // namespace

FG_API int fg_bpat_save(fg_ctx *ctx, const char *path, int header, int n,
                        const fg_bpat_tensor *tensors) {
    FG_REQUIRE(ctx, FG_ERR_INVALID_ARGUMENT, "fg_bpat_save: ctx is NULL");
    FG_HIP(hipSetDevice(ctx->device));
    auto fetch = [&](const fg_bpat_tensor &T, std::vector<uint8_t> &raw) -> int {
        FG_HIP(hipMemcpyAsync(raw.data(), T.d_ptr, raw.size(), hipMemcpyDeviceToHost,
                              ctx->stream));
        FG_HIP(hipStreamSynchronize(ctx->stream));
        return FG_OK;
    };
    return save_impl(path, header, n, tensors, fetch, "fg_bpat_save");
}

FG_API int fg_bpat_save_host(const char *path, int header, int n,
                             const fg_bpat_tensor *tensors) {
    auto fetch = [](const fg_bpat_tensor &T, std::vector<uint8_t> &raw) -> int {
        std::memcpy(raw.data(), T.d_ptr, raw.size());
        return FG_OK;
    };
    return save_impl(path, header, n, tensors, fetch, "fg_bpat_save_host");
}

FG_API int fg_bpat_open(const char *path, fg_bpat **out) {
    FG_REQUIRE(path && out, FG_ERR_INVALID_ARGUMENT, "fg_bpat_open: NULL argument");
    FILE *fp = std::fopen(path, "rb");
    if (!fp) {
        fg::set_error("bpat %s: no such file", path);
        return FG_ERR_FILE_NOT_FOUND;
    }
    std::unique_ptr<fg_bpat> f(new fg_bpat);
    uint8_t buf[1 << 16];
    size_t got;
    while ((got = std::fread(buf, 1, sizeof buf, fp)) > 0) f->image.insert(f->image.end(), buf, buf + got);
    const bool err = std::ferror(fp) != 0;
    std::fclose(fp);
    if (err) return serial_err("read failed", path);
    const int rc = parse(*f, path);
    if (rc) return rc;
    *out = f.release();
    return FG_OK;
}

FG_API int fg_bpat_close(fg_bpat *f) {
    delete f;
    return FG_OK;
}

FG_API int fg_bpat_info(const fg_bpat *f, int *header, int *count) {
    FG_REQUIRE(f, FG_ERR_INVALID_ARGUMENT, "fg_bpat_info: NULL file");
    if (header) *header = f->header;
    if (count) *count = (int)f->tensors.size();
    return FG_OK;
}

FG_API int fg_bpat_tensor_info(const fg_bpat *f, int index, int *rank, uint32_t *shape,
                               uint64_t *numel) {
    FG_REQUIRE(f, FG_ERR_INVALID_ARGUMENT, "fg_bpat_tensor_info: NULL file");
    FG_REQUIRE(index >= 0 && index < (int)f->tensors.size(), FG_ERR_OUT_OF_BOUNDS,
               "fg_bpat_tensor_info: tensor %d of %zu", index, f->tensors.size());
    const FileTensor &t = f->tensors[index];
    if (rank) *rank = t.rank;
    if (shape)
        for (int d = 0; d < t.rank; ++d) shape[d] = t.shape[d];
    if (numel) *numel = t.numel;
    return FG_OK;
}

FG_API int fg_bpat_read_f32(const fg_bpat *f, int index, float *dst) {
    FG_REQUIRE(f && dst, FG_ERR_INVALID_ARGUMENT, "fg_bpat_read_f32: NULL argument");
    FG_REQUIRE(index >= 0 && index < (int)f->tensors.size(), FG_ERR_OUT_OF_BOUNDS,
               "fg_bpat_read_f32: tensor %d of %zu", index, f->tensors.size());
    const FileTensor &t = f->tensors[index];
    convert(f->image.data() + t.offset, kFormats[f->header].elem, reinterpret_cast<uint8_t *>(dst),
            kE32, t.numel);
    return FG_OK;
}

FG_API int fg_bpat_upload(fg_ctx *ctx, const fg_bpat *f, int index, void *d_dst, int dtype) {
    FG_REQUIRE(ctx && f && d_dst, FG_ERR_INVALID_ARGUMENT, "fg_bpat_upload: NULL argument");
    FG_REQUIRE(dtype >= FG_DTYPE_F32 && dtype <= FG_DTYPE_BF16, FG_ERR_INVALID_ARGUMENT,
               "fg_bpat_upload: unknown dtype %d", dtype);
    FG_REQUIRE(index >= 0 && index < (int)f->tensors.size(), FG_ERR_OUT_OF_BOUNDS,
               "fg_bpat_upload: tensor %d of %zu", index, f->tensors.size());
    const FileTensor &t = f->tensors[index];
    const int de = elem_of_dtype(dtype);
    std::vector<uint8_t> conv(t.numel * elem_bytes(de));
    convert(f->image.data() + t.offset, kFormats[f->header].elem, conv.data(), de, t.numel);
    if (conv.empty()) return FG_OK;
    FG_HIP(hipSetDevice(ctx->device));
    FG_HIP(hipMemcpyAsync(d_dst, conv.data(), conv.size(), hipMemcpyHostToDevice, ctx->stream));
    FG_HIP(hipStreamSynchronize(ctx->stream));
    return FG_OK;
}
