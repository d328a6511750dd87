// PNG pages to 8-bit RGB, written from the PNG specification (W3C PNG Second Edition, the same
// text as ISO/IEC 15948): chunk layout and CRC-32 (5.3), IHDR (11.2.2), PLTE (11.2.3), the IDAT
// chunks as one zlib stream (10), scanline filters (9.2), Adam7 passes (8.2). DEFLATE itself is
// zlib's raw inflate.
//
// The output is what the reference's page decode, image::open(p)?.into_rgb8()
// (src/bin/ocr-bench.rs:424; image 0.25.10 over png 0.18.1 in the reference's Cargo.lock), gives:
// grey replicated to R, G and B; alpha dropped, not blended; palette indices looked up, an index
// past the palette's end giving black (the png crate's 256-entry table); samples of 1, 2 or 4 bits
// scaled to 0..255 (x 255, 85, 17); 16-bit samples rounded to the nearest 8-bit value,
// round(v * 255 / 65535) = (v + 128) / 257. Chunk CRCs are checked; the zlib stream's Adler-32
// trailer is not (png 0.18 ignores it by default).
#include "png.h"

#include <zlib.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace ocr {
namespace {

const uint8_t kSignature[8] = {137, 80, 78, 71, 13, 10, 26, 10};

inline uint32_t be32(const uint8_t *p) {
    return uint32_t(p[0]) << 24 | uint32_t(p[1]) << 16 | uint32_t(p[2]) << 8 | uint32_t(p[3]);
}
constexpr uint32_t tag(const char (&s)[5]) {
    return uint32_t(uint8_t(s[0])) << 24 | uint32_t(uint8_t(s[1])) << 16 | uint32_t(uint8_t(s[2])) << 8 |
           uint32_t(uint8_t(s[3]));
}
std::string tag_name(uint32_t t) {
    std::string s(4, ' ');
    for (int i = 0; i < 4; i++) s[i] = char(t >> (24 - 8 * i));
    return s;
}

struct Chunk {
    uint32_t type = 0;
    const uint8_t *data = nullptr;
    uint32_t len = 0;
};

// The chunk at off, its CRC checked (over type and data); off moves past it.
Chunk read_chunk(const uint8_t *d, size_t n, size_t &off) {
    if (n - off < 12) fail("png: truncated chunk at byte " + std::to_string(off));
    Chunk c;
    c.len = be32(d + off);
    c.type = be32(d + off + 4);
    c.data = d + off + 8;
    if (c.len > 0x7fffffffu) fail("png: chunk length above 2^31 - 1");
    if (n - off - 12 < c.len) fail("png: truncated " + tag_name(c.type) + " chunk");
    for (int i = 0; i < 4; i++) {
        const uint8_t ch = uint8_t(c.type >> (24 - 8 * i)) | 0x20;
        if (ch < 'a' || ch > 'z') fail("png: invalid chunk type at byte " + std::to_string(off));
    }
    const uint32_t crc = uint32_t(crc32(0L, d + off + 4, uInt(c.len + 4)));
    if (crc != be32(c.data + c.len)) fail("png: CRC mismatch in the " + tag_name(c.type) + " chunk");
    off += 12 + size_t(c.len);
    return c;
}

int channels(int color) { return color == 0 || color == 3 ? 1 : color == 2 ? 3 : color == 4 ? 2 : 4; }

PngHeader parse_ihdr(const uint8_t *d, size_t n, size_t &off) {
    if (n < 8 || std::memcmp(d, kSignature, 8) != 0) fail("png: not a PNG file (signature)");
    off = 8;
    const Chunk c = read_chunk(d, n, off);
    if (c.type != tag("IHDR") || c.len != 13) fail("png: the first chunk is not a 13-byte IHDR");
    PngHeader h;
    h.w = be32(c.data);
    h.h = be32(c.data + 4);
    h.depth = c.data[8];
    h.color = c.data[9];
    h.interlace = c.data[12];
    if (h.w == 0 || h.h == 0 || h.w > 0x7fffffffu || h.h > 0x7fffffffu)
        fail("png: image size " + std::to_string(h.w) + " x " + std::to_string(h.h) + " out of range");
    const int dp = h.depth;
    bool ok = false;
    switch (h.color) {
    case 0: ok = dp == 1 || dp == 2 || dp == 4 || dp == 8 || dp == 16; break;
    case 3: ok = dp == 1 || dp == 2 || dp == 4 || dp == 8; break;
    case 2:
    case 4:
    case 6: ok = dp == 8 || dp == 16; break;
    }
    if (!ok) fail("png: colour type " + std::to_string(h.color) + " with bit depth " + std::to_string(dp));
    if (c.data[10] != 0) fail("png: compression method " + std::to_string(c.data[10]));
    if (c.data[11] != 0) fail("png: filter method " + std::to_string(c.data[11]));
    if (h.interlace > 1) fail("png: interlace method " + std::to_string(h.interlace));
    return h;
}

// The IDAT chunks' data as one zlib stream (RFC 1950 header, then raw DEFLATE), inflated on
// demand into the caller's buffers.
class Inflater {
  public:
    explicit Inflater(std::vector<Chunk> idat) : idat_(std::move(idat)) {
        const uint8_t cmf = next_byte(), flg = next_byte();
        if ((cmf & 15) != 8 || (cmf >> 4) > 7 || (unsigned(cmf) * 256 + flg) % 31 != 0 || (flg & 0x20))
            fail("png: bad zlib header in the image data");
        if (inflateInit2(&z_, -15) != Z_OK) fail("png: inflateInit2 failed");
    }
    ~Inflater() { inflateEnd(&z_); }
    Inflater(const Inflater &) = delete;
    Inflater &operator=(const Inflater &) = delete;

    // Exactly k bytes of the image data into dst.
    void read(uint8_t *dst, size_t k) {
        while (k) {
            const size_t step = k < (size_t(1) << 30) ? k : (size_t(1) << 30);
            z_.next_out = dst;
            z_.avail_out = uInt(step);
            while (z_.avail_out) {
                if (ended_) fail("png: image data truncated (the zlib stream ends early)");
                if (z_.avail_in == 0 && !refill()) fail("png: image data truncated");
                const int r = inflate(&z_, Z_NO_FLUSH);
                if (r == Z_STREAM_END) {
                    ended_ = true;
                } else if (r != Z_OK && !(r == Z_BUF_ERROR && z_.avail_in == 0)) {
                    fail(std::string("png: corrupt image data (") + (z_.msg ? z_.msg : "zlib error") + ")");
                }
            }
            dst += step;
            k -= step;
        }
    }

  private:
    uint8_t next_byte() {
        while (span_ < idat_.size() && pos_ == idat_[span_].len) {
            span_++;
            pos_ = 0;
        }
        if (span_ == idat_.size()) fail("png: image data truncated");
        return idat_[span_].data[pos_++];
    }
    bool refill() {
        while (span_ < idat_.size()) {
            const Chunk &c = idat_[span_++];
            const uint32_t from = pos_;
            pos_ = 0;
            if (c.len > from) {
                z_.next_in = const_cast<Bytef *>(c.data + from);
                z_.avail_in = uInt(c.len - from);
                return true;
            }
        }
        return false;
    }

    std::vector<Chunk> idat_;
    size_t span_ = 0;
    uint32_t pos_ = 0;
    z_stream z_{};
    bool ended_ = false;
};

inline uint8_t paeth(int a, int b, int c) {
    const int pa = std::abs(b - c), pb = std::abs(a - c), pc = std::abs(a + b - 2 * c);
    return uint8_t(pa <= pb && pa <= pc ? a : pb <= pc ? b : c);
}

// One scanline's filter undone (PNG 9.2): x[i] = raw[i] + predictor mod 256, the predictor built
// from a (the byte bpp to the left in this row), b (the byte above) and c (above and to the left),
// each zero outside the row. prior is the previous unfiltered row of the pass (zeros for its first
// row); raw and x may be the same buffer.
void unfilter(int type, const uint8_t *raw, uint8_t *x, const uint8_t *prior, size_t rb, size_t bpp) {
    switch (type) {
    case 0:
        if (raw != x) std::memcpy(x, raw, rb);
        return;
    case 1:
        for (size_t i = 0; i < bpp; i++) x[i] = raw[i];
        for (size_t i = bpp; i < rb; i++) x[i] = uint8_t(raw[i] + x[i - bpp]);
        return;
    case 2:
        for (size_t i = 0; i < rb; i++) x[i] = uint8_t(raw[i] + prior[i]);
        return;
    case 3:
        for (size_t i = 0; i < bpp; i++) x[i] = uint8_t(raw[i] + (prior[i] >> 1));
        for (size_t i = bpp; i < rb; i++) x[i] = uint8_t(raw[i] + ((x[i - bpp] + prior[i]) >> 1));
        return;
    case 4:
        for (size_t i = 0; i < bpp; i++) x[i] = uint8_t(raw[i] + prior[i]);
        for (size_t i = bpp; i < rb; i++) x[i] = uint8_t(raw[i] + paeth(x[i - bpp], prior[i], prior[i - bpp]));
        return;
    default: fail("png: unknown filter type " + std::to_string(type));
    }
}

// Unfiltered scanlines of any colour type and depth to RGB triples in the output image.
struct Emitter {
    PngHeader h;
    uint8_t pal[256 * 3] = {};  // entries past the PLTE stay black
    uint8_t *out = nullptr;

    static uint8_t s16(const uint8_t *s, size_t k) { return uint8_t(((unsigned(s[2 * k]) << 8 | s[2 * k + 1]) + 128) / 257); }
    static unsigned bits(const uint8_t *s, size_t i, int d) {
        const size_t b = i * size_t(d);
        return (s[b >> 3] >> (8 - d - int(b & 7))) & ((1u << d) - 1);
    }

    // Pixel i of the row s goes to column x0 + i * dx of output row y.
    void row(const uint8_t *s, uint32_t n, uint32_t y, uint32_t x0, uint32_t dx) const {
        uint8_t *o = out + (size_t(y) * h.w + x0) * 3;
        const size_t step = size_t(dx) * 3;
        const int d = h.depth;
        auto put = [&](uint32_t i, uint8_t r, uint8_t g, uint8_t b) {
            uint8_t *p = o + i * step;
            p[0] = r;
            p[1] = g;
            p[2] = b;
        };
        switch (h.color) {
        case 0:
            for (uint32_t i = 0; i < n; i++) {
                const uint8_t g = d == 16 ? s16(s, i) : d == 8 ? s[i] : uint8_t(bits(s, i, d) * (255u / ((1u << d) - 1)));
                put(i, g, g, g);
            }
            break;
        case 2:
            for (uint32_t i = 0; i < n; i++) {
                if (d == 8)
                    put(i, s[3 * i], s[3 * i + 1], s[3 * i + 2]);
                else
                    put(i, s16(s, 3 * i), s16(s, 3 * i + 1), s16(s, 3 * i + 2));
            }
            break;
        case 3:
            for (uint32_t i = 0; i < n; i++) {
                const unsigned v = d == 8 ? s[i] : bits(s, i, d);
                put(i, pal[3 * v], pal[3 * v + 1], pal[3 * v + 2]);
            }
            break;
        case 4:
            for (uint32_t i = 0; i < n; i++) {
                const uint8_t g = d == 8 ? s[2 * i] : s16(s, 2 * i);
                put(i, g, g, g);
            }
            break;
        case 6:
            for (uint32_t i = 0; i < n; i++) {
                if (d == 8)
                    put(i, s[4 * i], s[4 * i + 1], s[4 * i + 2]);
                else
                    put(i, s16(s, 4 * i), s16(s, 4 * i + 1), s16(s, 4 * i + 2));
            }
            break;
        }
    }
};

}  // namespace

PngHeader png_header(const uint8_t *data, size_t n) {
    if (!data) fail("png: null data");
    size_t off = 0;
    return parse_ihdr(data, n, off);
}

PngHeader png_decode_rgb(const uint8_t *data, size_t n, uint8_t *out, size_t cap) {
    if (!data || !out) fail("png: null buffer");
    size_t off = 0;
    Emitter em;
    em.h = parse_ihdr(data, n, off);
    em.out = out;
    const PngHeader &h = em.h;
    const size_t need = size_t(h.w) * h.h * 3;
    if (cap < need) fail("png: output buffer of " + std::to_string(cap) + " bytes; the image needs " + std::to_string(need));

    std::vector<Chunk> idat;
    bool have_pal = false, idat_closed = false;
    while (off < n) {
        const Chunk c = read_chunk(data, n, off);
        if (!idat.empty() && c.type != tag("IDAT")) idat_closed = true;
        if (c.type == tag("IEND")) break;
        if (c.type == tag("IDAT")) {
            if (idat_closed) fail("png: IDAT chunks are not consecutive");
            idat.push_back(c);
        } else if (c.type == tag("PLTE")) {
            if (!idat.empty()) fail("png: PLTE after the image data");
            if (have_pal) fail("png: second PLTE");
            if (c.len == 0 || c.len % 3 || c.len > 768) fail("png: PLTE of " + std::to_string(c.len) + " bytes");
            std::memcpy(em.pal, c.data, c.len);
            have_pal = true;
        } else if (c.type == tag("IHDR")) {
            fail("png: second IHDR");
        } else if (!(c.type & 0x20000000u)) {
            fail("png: unknown critical chunk " + tag_name(c.type));
        }
    }
    if (idat.empty()) fail("png: no image data");
    if (h.color == 3 && !have_pal) fail("png: palette image without PLTE");

    Inflater z(std::move(idat));
    const int ch = channels(h.color);
    const size_t bpp = size_t(ch * h.depth + 7) / 8;  // bytes a filter looks back (at least 1)
    if (h.interlace == 0 && h.color == 2 && h.depth == 8) {
        // RGB at 8 bits (every page the reference ships): the filter is undone straight into the
        // output, whose previous row is the prior.
        const size_t rb = size_t(h.w) * 3;
        std::vector<uint8_t> raw(rb + 1), zero(rb, 0);
        for (uint32_t y = 0; y < h.h; y++) {
            z.read(raw.data(), rb + 1);
            uint8_t *x = out + size_t(y) * rb;
            unfilter(raw[0], raw.data() + 1, x, y ? x - rb : zero.data(), rb, 3);
        }
        return h;
    }
    // Adam7 passes (x0, y0, dx, dy); a non-interlaced image is the single pass (0, 0, 1, 1).
    static const uint32_t kAdam7[7][4] = {{0, 0, 8, 8}, {4, 0, 8, 8}, {0, 4, 4, 8}, {2, 0, 4, 4},
                                          {0, 2, 2, 4}, {1, 0, 2, 2}, {0, 1, 1, 2}};
    static const uint32_t kWhole[1][4] = {{0, 0, 1, 1}};
    const uint32_t(*passes)[4] = h.interlace ? kAdam7 : kWhole;
    const int npass = h.interlace ? 7 : 1;
    const size_t max_rb = (size_t(h.w) * ch * h.depth + 7) / 8;
    std::vector<uint8_t> raw(max_rb + 1), cur(max_rb), prev(max_rb);
    for (int p = 0; p < npass; p++) {
        const uint32_t x0 = passes[p][0], y0 = passes[p][1], dx = passes[p][2], dy = passes[p][3];
        if (h.w <= x0 || h.h <= y0) continue;  // an empty pass has no scanlines at all
        const uint32_t pw = (h.w - x0 + dx - 1) / dx, ph = (h.h - y0 + dy - 1) / dy;
        const size_t rb = (size_t(pw) * ch * h.depth + 7) / 8;
        std::fill(prev.begin(), prev.begin() + rb, 0);
        for (uint32_t r = 0; r < ph; r++) {
            z.read(raw.data(), rb + 1);
            unfilter(raw[0], raw.data() + 1, cur.data(), prev.data(), rb, bpp);
            em.row(cur.data(), pw, y0 + r * dy, x0, dx);
            std::swap(cur, prev);
        }
    }
    return h;
}

}  // namespace ocr
