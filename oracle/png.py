"""ORACLE (test infrastructure only): PNG pages to 8-bit RGB, the oracle of the page decode
image::open(p)?.into_rgb8() (src/bin/ocr-bench.rs:424, src/bin/stages.rs:94,
src/bin/ppocr-bench.rs:69; image 0.25.10 over png 0.18.1 in the reference's Cargo.lock).

Neither crate is vendored, so this is restated from the PNG specification (W3C PNG Second
Edition = ISO/IEC 15948): chunk layout and CRC-32 (5.3), IHDR (11.2.2), PLTE (11.2.3), the IDAT
chunks as one zlib stream (10), the five scanline filters (9.2, Paeth as 9.4 writes it), Adam7
(8.2). DEFLATE is Python's zlib. The conversion is into_rgb8's: grey replicated to R, G and B,
alpha dropped (not blended), palette indices looked up (past the palette's end: black, the png
crate's 256-entry table), 1/2/4-bit samples scaled to 0..255, 16-bit samples to the nearest 8-bit
value.

Pinned (tests/test_png.py): against Pillow's decoder for every 8-bit and low-bit colour type,
palettes of 1-8 bits and Adam7; by encode -> decode round trips over every filter type; by the
nearest-value property of the 16-bit rescaling; and by the reference's own page PNGs
(data/pages, hashes in tests/golden/png_pages.json). Whether image 0.25 rounds 16-bit samples to
the nearest value (rather than truncating) is parity unpinned: neither crate is here to run.
Pure Python loops: small images only.
"""
from __future__ import annotations

import struct
import zlib

import numpy as np

SIGNATURE = b"\x89PNG\r\n\x1a\n"
ALLOWED_DEPTHS = {0: (1, 2, 4, 8, 16), 2: (8, 16), 3: (1, 2, 4, 8), 4: (8, 16), 6: (8, 16)}
CHANNELS = {0: 1, 2: 3, 3: 1, 4: 2, 6: 4}
# Adam7 passes: (first column, first row, column step, row step), PNG 8.2.
ADAM7 = [(0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2), (0, 1, 1, 2)]


class PngError(ValueError):
    pass


def chunks(data: bytes):
    """(type, body) of every chunk up to IEND, each CRC checked."""
    if data[:8] != SIGNATURE:
        raise PngError("signature")
    pos, out = 8, []
    while pos < len(data):
        if len(data) - pos < 12:
            raise PngError("truncated chunk")
        (n,) = struct.unpack(">I", data[pos:pos + 4])
        typ = data[pos + 4:pos + 8]
        if n > 2**31 - 1 or pos + 12 + n > len(data):
            raise PngError("truncated chunk")
        if not typ.isalpha():
            raise PngError("chunk type")
        body = data[pos + 8:pos + 8 + n]
        (crc,) = struct.unpack(">I", data[pos + 8 + n:pos + 12 + n])
        if zlib.crc32(typ + body) != crc:
            raise PngError("CRC")
        out.append((typ, body))
        pos += 12 + n
        if typ == b"IEND":
            break
    return out


def header(data: bytes):
    """(w, h, depth, colour type, interlace) from IHDR."""
    cs = chunks(data[:8 + 25]) if len(data) >= 33 else chunks(data)
    if not cs or cs[0][0] != b"IHDR" or len(cs[0][1]) != 13:
        raise PngError("IHDR")
    w, h, depth, color, comp, filt, inter = struct.unpack(">IIBBBBB", cs[0][1])
    if not (0 < w < 2**31 and 0 < h < 2**31) or depth not in ALLOWED_DEPTHS.get(color, ()) or comp or filt \
            or inter > 1:
        raise PngError("IHDR fields")
    return w, h, depth, color, inter


def _unfilter(ft: int, x: bytearray, prior: bytearray, bpp: int) -> None:
    """PNG 9.2: undo filter ft on the row x in place; prior is the previous unfiltered row."""
    if ft > 4:
        raise PngError("filter type")
    if ft == 0:
        return
    for i in range(len(x)):
        a = x[i - bpp] if i >= bpp else 0
        b = prior[i]
        c = prior[i - bpp] if i >= bpp else 0
        if ft == 1:
            pred = a
        elif ft == 2:
            pred = b
        elif ft == 3:
            pred = (a + b) // 2
        else:  # Paeth, as PNG 9.4 states it
            p = a + b - c
            pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
            pred = a if (pa <= pb and pa <= pc) else (b if pb <= pc else c)
        x[i] = (x[i] + pred) % 256


def _samples(row: bytes, n: int, depth: int) -> np.ndarray:
    """The first n samples of an unfiltered row as integers."""
    a = np.frombuffer(bytes(row), np.uint8)
    if depth == 8:
        return a[:n].astype(np.int64)
    if depth == 16:
        return a.view(">u2")[:n].astype(np.int64)
    bits = np.unpackbits(a)[: n * depth].reshape(n, depth).astype(np.int64)
    return bits @ (1 << np.arange(depth - 1, -1, -1))


def to8(v: np.ndarray, depth: int) -> np.ndarray:
    """Samples of `depth` bits to 0..255: exact multiples below 8 bits; 16 bits to the nearest
    value, v * 255 / 65535 rounded half up in exact integer arithmetic."""
    if depth == 16:
        return (v * 255 * 2 + 65535) // (2 * 65535)
    return v * 255 // ((1 << depth) - 1)


def decode_rgb(data: bytes) -> np.ndarray:
    """The whole image as an [h, w, 3] uint8 array."""
    cs = chunks(data)
    w, h, depth, color, inter = header(data)
    palette, idat, closed = None, [], False
    for typ, body in cs[1:]:
        if idat and typ != b"IDAT":
            closed = True
        if typ == b"IEND":
            break
        if typ == b"IDAT":
            if closed:
                raise PngError("IDAT not consecutive")
            idat.append(body)
        elif typ == b"PLTE":
            if idat or palette is not None or not body or len(body) % 3 or len(body) > 768:
                raise PngError("PLTE")
            palette = np.zeros((256, 3), np.int64)
            palette[: len(body) // 3] = np.frombuffer(body, np.uint8).reshape(-1, 3)
        elif typ == b"IHDR":
            raise PngError("second IHDR")
        elif not typ[0] & 0x20:
            raise PngError("unknown critical chunk")
    if not idat:
        raise PngError("no image data")
    if color == 3 and palette is None:
        raise PngError("no PLTE")
    stream = b"".join(idat)
    if len(stream) < 2:
        raise PngError("truncated")
    cmf, flg = stream[0], stream[1]
    if cmf & 15 != 8 or cmf >> 4 > 7 or (cmf * 256 + flg) % 31 or flg & 0x20:
        raise PngError("zlib header")
    try:
        raw = zlib.decompressobj(-15).decompress(stream[2:])
    except zlib.error as e:
        raise PngError(f"corrupt image data: {e}") from e

    ch = CHANNELS[color]
    bpp = max(1, ch * depth // 8)
    out = np.zeros((h, w, 3), np.uint8)
    off = 0
    for x0, y0, dx, dy in ADAM7 if inter else [(0, 0, 1, 1)]:
        if w <= x0 or h <= y0:
            continue
        pw, ph = (w - x0 + dx - 1) // dx, (h - y0 + dy - 1) // dy
        rb = (pw * ch * depth + 7) // 8
        prior = bytearray(rb)
        for r in range(ph):
            if off + 1 + rb > len(raw):
                raise PngError("truncated image data")
            ft, x = raw[off], bytearray(raw[off + 1:off + 1 + rb])
            off += 1 + rb
            _unfilter(ft, x, prior, bpp)
            s = _samples(x, pw * ch, depth).reshape(pw, ch)
            if color == 3:
                rgb = palette[s[:, 0]]
            elif color in (0, 4):
                rgb = np.repeat(to8(s[:, :1], depth), 3, axis=1)
            else:
                rgb = to8(s[:, :3], depth)
            out[y0 + r * dy, x0::dx] = rgb.astype(np.uint8)
            prior = x
    return out
