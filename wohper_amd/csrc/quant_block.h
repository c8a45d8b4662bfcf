// ZCBLK01 quant-block reader (host code, no HIP): the expert blocks the
// engine reads from its model files, parsed in place into byte ranges that
// the weight store uploads.  Follows the reference's parser check for check,
// in the same order, so a malformed block fails with the same error:
//   parse_quant_block               E/compute.rs:1099-1148
//   QuantBlockLayout::tensor        E/compute.rs:545-600
//   read_name_blob / read_shape_layout / read_le_bytes
//                                   E/compute.rs:7136-7178, 7200-7213
//   find_tensor_by_suffix           E/compute.rs:1150-1169
//   deepseek_fp4_matvec_from_tensors E/compute.rs:1201-1247
//   deepseek_v4_fp4_expert_from_quant_block E/compute.rs:1249-1268
// Block layout (little endian): a 40-byte header {magic "ZCBLK01\0",
// u32 version = 1, u32 tensor_count, u32 quant_format, u32 flags,
// u64 record_table_offset, u64 names_offset}; tensor_count 52-byte records
// {u16 dtype_original, u16 quant_format, u32 rank, u32 flags,
// u64 name_offset, u64 shape_offset, u64 data_offset, u64 data_bytes,
// f32 scale, f32 zero_point}; names are {u16 len, bytes} at
// names_offset + name_offset; shapes are {u32 rank, rank x u64} at
// shape_offset.  Offsets are absolute except name_offset.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>

namespace whqb {

constexpr size_t kHeaderBytes = 40;
constexpr size_t kRecordBytes = 52;
constexpr uint32_t kVersion = 1;
constexpr uint16_t kQuantFp4 = 2402;  // E/deepseek_v4.rs:41-47
constexpr uint16_t kQuantUe8m0 = 2403;

// Error classes of ComputeError (E/compute.rs:330-344) that the reader can
// raise, with the reference's static detail text.
enum class Fail : int {
    None = 0,
    Truncated,       // TruncatedQuantBlock(field)
    Magic,           // InvalidQuantBlockMagic(magic)
    Version,         // UnsupportedQuantBlockVersion(version)
    Invalid,         // InvalidQuantBlock(reason)
    Shape,           // InvalidShape(name)
};

struct Error {
    Fail kind = Fail::None;
    const char* what = "";
    uint8_t magic[8] = {};
    uint32_t version = 0;
};

// The reference's Display text of an error (E/compute.rs:346-372).
inline void describe(const Error& e, char* out, size_t n) {
    switch (e.kind) {
        case Fail::None: std::snprintf(out, n, "ok"); break;
        case Fail::Truncated: std::snprintf(out, n, "truncated ZCBLK field: %s", e.what); break;
        case Fail::Magic:
            std::snprintf(out, n, "invalid ZCBLK magic: [%u, %u, %u, %u, %u, %u, %u, %u]", e.magic[0], e.magic[1],
                          e.magic[2], e.magic[3], e.magic[4], e.magic[5], e.magic[6], e.magic[7]);
            break;
        case Fail::Version: std::snprintf(out, n, "unsupported ZCBLK version: %u", e.version); break;
        case Fail::Invalid: std::snprintf(out, n, "invalid ZCBLK: %s", e.what); break;
        case Fail::Shape: std::snprintf(out, n, "invalid compute shape: %s", e.what); break;
    }
}

// a + b, false on wrap-around (the reference's checked_add).
inline bool add_ok(size_t a, size_t b, size_t* r) { return !__builtin_add_overflow(a, b, r); }
inline bool mul_ok(size_t a, size_t b, size_t* r) { return !__builtin_mul_overflow(a, b, r); }

class Reader {
public:
    Reader(const uint8_t* buf, size_t len) : buf_(buf), len_(len) {}

    // Little-endian field of N bytes at `off`; a range past the end is
    // TruncatedQuantBlock(field), one that wraps is "read range overflow".
    template <class T>
    bool get(size_t off, const char* field, T* v, Error* err) const {
        size_t end;
        if (!add_ok(off, sizeof(T), &end)) return fail(err, Fail::Invalid, "read range overflow");
        if (end > len_) return fail(err, Fail::Truncated, field);
        std::memcpy(v, buf_ + off, sizeof(T));  // the host is little endian (x86-64)
        return true;
    }
    // [off, off + n) inside the buffer.
    bool span(size_t off, size_t n, const char* overflow, const char* field, Error* err) const {
        size_t end;
        if (!add_ok(off, n, &end)) return fail(err, Fail::Invalid, overflow);
        if (end > len_) return fail(err, Fail::Truncated, field);
        return true;
    }
    size_t size() const { return len_; }
    const uint8_t* data() const { return buf_; }

    static bool fail(Error* err, Fail kind, const char* what) {
        err->kind = kind;
        err->what = what;
        return false;
    }

private:
    const uint8_t* buf_;
    size_t len_;
};

struct Header {
    uint32_t tensor_count = 0, quant_format = 0, flags = 0;
    size_t record_table_offset = 0, names_offset = 0;
};

// One tensor record resolved against the buffer: name, shape and data are
// byte ranges of the block.
struct Tensor {
    uint16_t dtype_original = 0, quant_format = 0;
    uint32_t rank = 0, flags = 0;
    size_t name_off = 0, name_len = 0;
    size_t shape_off = 0;  // the {u32 rank, dims} blob
    size_t data_off = 0, data_len = 0;
    float scale = 0.f, zero_point = 0.f;

    uint64_t dim(const Reader& r, uint32_t i) const {
        uint64_t v = 0;
        std::memcpy(&v, r.data() + shape_off + 4 + 8 * (size_t)i, 8);
        return v;
    }
    bool name_ends_with(const Reader& r, const char* suffix) const {
        const size_t n = std::strlen(suffix);
        return name_len >= n && std::memcmp(r.data() + name_off + name_len - n, suffix, n) == 0;
    }
};

inline bool parse_header(const Reader& r, Header* h, Error* err) {
    static const uint8_t kMagic[8] = {'Z', 'C', 'B', 'L', 'K', '0', '1', 0};
    if (r.size() < kHeaderBytes) return Reader::fail(err, Fail::Truncated, "block header");
    if (std::memcmp(r.data(), kMagic, 8) != 0) {
        std::memcpy(err->magic, r.data(), 8);
        return Reader::fail(err, Fail::Magic, "");
    }
    uint32_t version = 0;
    uint64_t rto = 0, nmo = 0;
    r.get(8, "block.version", &version, err);
    if (version != kVersion) {
        err->version = version;
        return Reader::fail(err, Fail::Version, "");
    }
    r.get(12, "block.tensor_count", &h->tensor_count, err);
    r.get(16, "block.quant_format", &h->quant_format, err);
    r.get(20, "block.flags", &h->flags, err);
    r.get(24, "block.record_table_offset", &rto, err);
    r.get(32, "block.names_offset", &nmo, err);
    h->record_table_offset = (size_t)rto;
    h->names_offset = (size_t)nmo;
    size_t table_bytes, table_end;
    if (!mul_ok((size_t)h->tensor_count, kRecordBytes, &table_bytes))
        return Reader::fail(err, Fail::Invalid, "record table size overflow");
    if (!add_ok(h->record_table_offset, table_bytes, &table_end))
        return Reader::fail(err, Fail::Invalid, "record table range overflow");
    if (h->record_table_offset < kHeaderBytes || table_end > r.size())
        return Reader::fail(err, Fail::Truncated, "record table");
    if (h->names_offset > r.size()) return Reader::fail(err, Fail::Truncated, "names blob");
    return true;
}

// Record `index` (< tensor_count) with its name, shape and data ranges
// checked against the buffer.
inline bool tensor_at(const Reader& r, const Header& h, size_t index, Tensor* t, Error* err) {
    // the record lies inside the table parse_header bounded
    const size_t rec = h.record_table_offset + index * kRecordBytes;
    uint64_t name_rel = 0, shape_off = 0, data_off = 0, data_len = 0;
    r.get(rec + 0, "record.dtype_original", &t->dtype_original, err);
    r.get(rec + 2, "record.quant_format", &t->quant_format, err);
    r.get(rec + 4, "record.rank", &t->rank, err);
    r.get(rec + 8, "record.flags", &t->flags, err);
    r.get(rec + 12, "record.name_offset", &name_rel, err);
    r.get(rec + 20, "record.shape_offset", &shape_off, err);
    r.get(rec + 28, "record.data_offset", &data_off, err);
    r.get(rec + 36, "record.data_bytes", &data_len, err);
    r.get(rec + 44, "record.scale", &t->scale, err);
    r.get(rec + 48, "record.zero_point", &t->zero_point, err);

    // name: u16 length + bytes at names_offset + name_offset
    size_t at;
    if (!add_ok(h.names_offset, (size_t)name_rel, &at)) return Reader::fail(err, Fail::Invalid, "name offset overflow");
    uint16_t name_len = 0;
    if (!r.get(at, "name.len", &name_len, err)) return false;
    if (!r.span(at + 2, name_len, "name end overflow", "name blob", err)) return false;
    t->name_off = at + 2;
    t->name_len = name_len;

    // shape: u32 rank (must equal the record's) + rank x u64
    uint32_t rank = 0;
    if (!r.get((size_t)shape_off, "shape.rank", &rank, err)) return false;
    if (rank != t->rank) return Reader::fail(err, Fail::Invalid, "shape rank mismatch");
    if (!r.span((size_t)shape_off, 4 + 8 * (size_t)rank, "shape end overflow", "shape blob", err)) return false;
    t->shape_off = (size_t)shape_off;

    if (!r.span((size_t)data_off, (size_t)data_len, "tensor data range overflow", "tensor data", err)) return false;
    t->data_off = (size_t)data_off;
    t->data_len = (size_t)data_len;
    return true;
}

// The one tensor whose name ends with `suffix`; every record before the
// match (and up to a duplicate) must itself be well formed.
inline bool find_suffix(const Reader& r, const Header& h, const char* suffix, Tensor* out, Error* err) {
    bool found = false;
    for (size_t i = 0; i < h.tensor_count; ++i) {
        Tensor t;
        if (!tensor_at(r, h, i, &t, err)) return false;
        if (!t.name_ends_with(r, suffix)) continue;
        if (found) return Reader::fail(err, Fail::Invalid, "duplicate DeepSeek expert tensor suffix");
        *out = t;
        found = true;
    }
    if (!found) return Reader::fail(err, Fail::Invalid, "missing DeepSeek expert tensor suffix");
    return true;
}

// One FP4 projection: packed weight [rows][cols/2] + UE8M0 scales
// [rows][scale_cols], as byte ranges of the block.
struct Fp4 {
    size_t rows = 0, cols = 0, scale_cols = 0;
    size_t weight_off = 0, weight_len = 0;
    size_t scale_off = 0, scale_len = 0;
};

inline bool fp4_projection(const Reader& r, const Tensor& w, const Tensor& s, Fp4* p, Error* err) {
    if (w.quant_format != kQuantFp4)
        return Reader::fail(err, Fail::Invalid, "DeepSeek expert weight is not FP4 E2M1 packed");
    if (s.quant_format != kQuantUe8m0) return Reader::fail(err, Fail::Invalid, "DeepSeek expert scale is not UE8M0");
    if (w.rank != 2 || s.rank != 2) return Reader::fail(err, Fail::Shape, "DeepSeek FP4 expert rank");
    const size_t rows = (size_t)w.dim(r, 0), packed = (size_t)w.dim(r, 1);
    const size_t srows = (size_t)s.dim(r, 0), scols = (size_t)s.dim(r, 1);
    if (rows == 0 || packed == 0 || scols == 0 || srows != rows)
        return Reader::fail(err, Fail::Shape, "DeepSeek FP4 expert shape");
    size_t cols, wbytes, sbytes;
    if (!mul_ok(packed, 2, &cols)) return Reader::fail(err, Fail::Shape, "DeepSeek FP4 expert cols overflow");
    if (!mul_ok(rows, packed, &wbytes)) return Reader::fail(err, Fail::Shape, "DeepSeek FP4 expert weight overflow");
    if (w.data_len < wbytes) return Reader::fail(err, Fail::Truncated, "DeepSeek FP4 expert weight");
    if (!mul_ok(rows, scols, &sbytes)) return Reader::fail(err, Fail::Shape, "DeepSeek FP4 expert scale overflow");
    if (s.data_len < sbytes) return Reader::fail(err, Fail::Truncated, "DeepSeek FP4 expert scale");
    p->rows = rows;
    p->cols = cols;
    p->scale_cols = scols;
    p->weight_off = w.data_off;
    p->weight_len = wbytes;
    p->scale_off = s.data_off;
    p->scale_len = sbytes;
    return true;
}

// The FP4 SwiGLU expert of a block: out[0] = w1 (gate), out[1] = w3 (up),
// out[2] = w2 (down).
inline bool fp4_expert(const uint8_t* buf, size_t len, Fp4 out[3], Error* err) {
    static const char* const kSuffix[3][2] = {
        {".w1.weight", ".w1.scale"}, {".w3.weight", ".w3.scale"}, {".w2.weight", ".w2.scale"}};
    Reader r(buf, len);
    Header h;
    if (!parse_header(r, &h, err)) return false;
    for (int m = 0; m < 3; ++m) {
        Tensor w, s;
        if (!find_suffix(r, h, kSuffix[m][0], &w, err)) return false;
        if (!find_suffix(r, h, kSuffix[m][1], &s, err)) return false;
        if (!fp4_projection(r, w, s, &out[m], err)) return false;
    }
    if (out[0].cols != out[1].cols || out[0].rows != out[1].rows || out[2].cols != out[0].rows)
        return Reader::fail(err, Fail::Shape, "DeepSeek FP4 expert projection");
    return true;
}

}  // namespace whqb
