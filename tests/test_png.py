"""PNG page decode (ocr_png_dims / ocr_png_decode; the reference's image::open(p)?.into_rgb8(),
src/bin/ocr-bench.rs:424), host only.

Pins of the oracle (oracle/png.py):
- Pillow, an independent decoder: every colour type at 8 bits and below (grey 1/2/4/8, RGB, palette
  1/2/4/8, grey + alpha, RGBA), plain and Adam7, odd sizes with empty Adam7 passes, files written
  here with every filter type and split IDAT chunks, and files Pillow itself writes;
- round trips: 8-bit RGB samples encoded under each filter come back unchanged;
- 16-bit samples: every value 0..65535 maps to its nearest 8-bit value (|257 * out - v| <= 128),
  and multiples of 257 map exactly;
- the reference's own page PNGs (data/pages) against Pillow's pixels (tests/golden/png_pages.json).
Then the library against the oracle on all of these, and the malformed files both must refuse.
"""
import glob
import hashlib
import io
import json
import os
import struct
import zlib

import numpy as np
import pytest

import ocrhip
from oracle import png as op

Image = pytest.importorskip("PIL.Image")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "png_pages.json")
PAGES = "/root/reference/data/pages"


# ---- a PNG writer for the tests: explicit filter types, Adam7, IDAT splits ------------------
def _chunk(typ: bytes, body: bytes) -> bytes:
    return struct.pack(">I", len(body)) + typ + body + struct.pack(">I", zlib.crc32(typ + body))


def _pack(samples: np.ndarray, depth: int) -> bytes:
    s = samples.astype(np.int64).reshape(-1)
    if depth == 8:
        return s.astype(np.uint8).tobytes()
    if depth == 16:
        return s.astype(">u2").tobytes()
    bits = (s[:, None] >> np.arange(depth - 1, -1, -1)) & 1
    return np.packbits(bits.astype(np.uint8).reshape(-1)).tobytes()


def _filter(ft: int, cur: bytes, prior: bytes, bpp: int) -> bytes:
    out = bytearray(len(cur))
    for i in range(len(cur)):
        a = cur[i - bpp] if i >= bpp else 0
        b = prior[i]
        c = prior[i - bpp] if i >= bpp else 0
        if ft == 0:
            pred = 0
        elif ft == 1:
            pred = a
        elif ft == 2:
            pred = b
        elif ft == 3:
            pred = (a + b) >> 1
        else:
            p = a + b - c
            pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
            pred = a if pa <= pb and pa <= pc else b if pb <= pc else c
        out[i] = (cur[i] - pred) & 255
    return bytes(out)


def encode(samples, color, depth, interlace=0, filters=(0, 1, 2, 3, 4), palette=None, split=None, level=6,
           before_idat=(), between_idat=b"", raw_tail=0):
    """samples: [h, w, channels] integers below 2^depth. filters: the filter type of each scanline in
    turn (cycled). split: IDAT chunk size. raw_tail: bytes dropped from the end of the image data."""
    h, w, ch = samples.shape
    bpp = max(1, ch * depth // 8)
    raw, k = bytearray(), 0
    for x0, y0, dx, dy in op.ADAM7 if interlace else [(0, 0, 1, 1)]:
        sub = samples[y0::dy, x0::dx]
        if sub.size == 0:
            continue
        prior = bytes(len(_pack(sub[0], depth)))
        for r in range(sub.shape[0]):
            cur = _pack(sub[r], depth)
            ft = filters[k % len(filters)]
            k += 1
            raw.append(ft)
            raw += _filter(min(ft, 4), cur, prior, bpp)
            prior = cur
    if raw_tail:
        raw = raw[:-raw_tail]
    data = zlib.compress(bytes(raw), level)
    out = b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, depth, color, 0, 0, interlace))
    if palette is not None:
        out += _chunk(b"PLTE", np.asarray(palette, np.uint8).tobytes())
    for typ, body in before_idat:
        out += _chunk(typ, body)
    parts = [data] if not split else [data[i:i + split] for i in range(0, len(data), split)]
    for i, p in enumerate(parts):
        out += _chunk(b"IDAT", p)
        if i == 0 and between_idat and len(parts) > 1:
            out += _chunk(between_idat, b"x")
    return out + _chunk(b"IEND", b"")


COMBOS = [(0, 1), (0, 2), (0, 4), (0, 8), (2, 8), (3, 1), (3, 2), (3, 4), (3, 8), (4, 8), (6, 8)]
COMBOS16 = [(0, 16), (2, 16), (4, 16), (6, 16)]
SIZES = [(1, 1), (3, 2), (2, 5), (5, 7), (8, 8), (17, 9), (33, 4)]


def _case(color, depth, w, h, seed):
    rng = np.random.default_rng(seed)
    ch = op.CHANNELS[color]
    samples = rng.integers(0, 1 << depth, size=(h, w, ch))
    palette = None
    if color == 3:
        n = 1 << depth
        palette = rng.integers(0, 256, size=(n, 3))
    return samples, palette


def _cases(combos):
    out = []
    for ci, (color, depth) in enumerate(combos):
        for si, (w, h) in enumerate(SIZES):
            for inter in (0, 1):
                seed = 1000 * ci + 10 * si + inter
                samples, palette = _case(color, depth, w, h, seed)
                filters = [(seed + j) % 5 for j in range(5)] if si % 2 else [4, 3, 1, 2, 0]
                split = [None, 1, 3, 64][si % 4]
                png = encode(samples, color, depth, inter, filters, palette, split=split)
                out.append((f"c{color}d{depth}_{w}x{h}_i{inter}", png, samples, palette))
    return out


CASES = _cases(COMBOS)
CASES16 = _cases(COMBOS16)


def _pil(png: bytes) -> np.ndarray:
    with Image.open(io.BytesIO(png)) as im:
        return np.asarray(im.convert("RGB"))


# ---- the oracle, pinned ------------------------------------------------------------------------
@pytest.mark.parametrize("name,png,samples,palette", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_pillow(name, png, samples, palette):
    np.testing.assert_array_equal(op.decode_rgb(png), _pil(png))


def test_oracle_rgb8_round_trip_every_filter():
    rng = np.random.default_rng(7)
    samples = rng.integers(0, 256, size=(6, 11, 3))
    for ft in range(5):
        for inter in (0, 1):
            png = encode(samples, 2, 8, inter, filters=(ft,))
            np.testing.assert_array_equal(op.decode_rgb(png), samples.astype(np.uint8))


def test_oracle_paeth_ties():
    """Samples 0..3 under the Paeth filter: the predictor's distance ties (pa = pb, pb = pc) are
    common, so the order in which it breaks them is exercised."""
    rng = np.random.default_rng(17)
    samples = rng.integers(0, 4, size=(24, 24, 3))
    for inter in (0, 1):
        png = encode(samples, 2, 8, inter, filters=(4,))
        np.testing.assert_array_equal(op.decode_rgb(png), samples.astype(np.uint8))
        np.testing.assert_array_equal(op.decode_rgb(png), _pil(png))
        np.testing.assert_array_equal(ocrhip.decode_png(png), samples.astype(np.uint8))


def test_oracle_pillow_written_files():
    rng = np.random.default_rng(3)
    for mode, shape in (("L", (37, 21)), ("RGB", (19, 40, 3)), ("RGBA", (23, 9, 4)), ("LA", (12, 30, 2)),
                        ("1", (17, 25))):
        a = rng.integers(0, 256, size=shape).astype(np.uint8)
        im = Image.fromarray(a if mode != "1" else a > 127, mode if mode != "1" else None)
        if mode == "1":
            im = im.convert("1")
        for level in (0, 9):
            buf = io.BytesIO()
            im.save(buf, "PNG", compress_level=level)
            png = buf.getvalue()
            np.testing.assert_array_equal(op.decode_rgb(png), _pil(png))
    p = Image.fromarray(rng.integers(0, 16, size=(14, 27)).astype(np.uint8), "L").convert("P")
    p.putpalette(list(rng.integers(0, 256, size=16 * 3)))
    for bits in (4, 8):
        buf = io.BytesIO()
        p.save(buf, "PNG", bits=bits)
        np.testing.assert_array_equal(op.decode_rgb(buf.getvalue()), _pil(buf.getvalue()))


def test_oracle_16bit_nearest():
    v = np.arange(65536).reshape(256, 256, 1)
    png = encode(v, 0, 16, filters=(0,))
    out = op.decode_rgb(png)[:, :, 0].astype(np.int64).reshape(-1)
    assert np.abs(257 * out - np.arange(65536)).max() <= 128
    k = np.arange(256).reshape(16, 16, 1) * 257
    rgb = np.concatenate([k, k[::-1], k.transpose(1, 0, 2)], axis=2)
    png = encode(rgb, 2, 16, interlace=1)
    np.testing.assert_array_equal(op.decode_rgb(png), (rgb // 257).astype(np.uint8))


def test_oracle_reference_pages():
    if not os.path.isdir(PAGES):
        pytest.skip("the reference's data/pages is not present")
    golden = json.load(open(GOLDEN))
    # Two small pages through the (slow, pure Python) oracle; all pages through the library below.
    for name in ("A_150/Text_page_4.png",):
        rgb = op.decode_rgb(open(os.path.join(PAGES, name), "rb").read())
        assert hashlib.sha256(rgb.tobytes()).hexdigest() == golden[name]["sha256"]


# ---- the library against the oracle --------------------------------------------------------------
@pytest.mark.parametrize("name,png,samples,palette", CASES + CASES16, ids=[c[0] for c in CASES + CASES16])
def test_png_decode_matches_oracle(name, png, samples, palette):
    h, w = samples.shape[:2]
    assert ocrhip.png_dims(png) == (w, h)
    np.testing.assert_array_equal(ocrhip.decode_png(png), op.decode_rgb(png))


def test_png_palette_index_past_end_is_black():
    samples = np.arange(16).reshape(4, 4, 1)
    png = encode(samples, 3, 4, palette=[[10, 20, 30], [40, 50, 60], [70, 80, 90]])
    got = ocrhip.decode_png(png)
    np.testing.assert_array_equal(got, op.decode_rgb(png))
    assert (got.reshape(-1, 3)[3:] == 0).all() and tuple(got[0, 1]) == (40, 50, 60)


def test_png_ancillary_chunks_and_level0():
    rng = np.random.default_rng(5)
    samples = rng.integers(0, 256, size=(9, 14, 4))
    png = encode(samples, 6, 8, 1, level=0, before_idat=[(b"tEXt", b"Title\x00page"), (b"gAMA", b"\x00\x01\x86\xa0"),
                                                         (b"zzZz", b"private")])
    np.testing.assert_array_equal(ocrhip.decode_png(png), samples[:, :, :3].astype(np.uint8))
    np.testing.assert_array_equal(op.decode_rgb(png), samples[:, :, :3].astype(np.uint8))


def _malformed():
    rng = np.random.default_rng(11)
    s = rng.integers(0, 256, size=(6, 7, 3))
    good = encode(s, 2, 8, split=20)
    idat = good.index(b"IDAT")
    bad = {}
    bad["signature"] = b"\x88" + good[1:]
    flip = bytearray(good)
    flip[idat + 6] ^= 1
    bad["crc"] = bytes(flip)
    bad["truncated_file"] = good[:idat + 10]
    bad["filter_type_5"] = encode(s, 2, 8, filters=(0, 5))
    bad["depth_4_rgb"] = good[:8] + _chunk(b"IHDR", struct.pack(">IIBBBBB", 7, 6, 4, 2, 0, 0, 0)) + good[33:]
    bad["interlace_2"] = good[:8] + _chunk(b"IHDR", struct.pack(">IIBBBBB", 7, 6, 8, 2, 0, 0, 2)) + good[33:]
    bad["zero_width"] = good[:8] + _chunk(b"IHDR", struct.pack(">IIBBBBB", 0, 6, 8, 2, 0, 0, 0)) + good[33:]
    bad["no_plte"] = encode(rng.integers(0, 4, size=(3, 3, 1)), 3, 2)
    bad["idat_not_consecutive"] = encode(s, 2, 8, split=10, between_idat=b"tEXt")
    bad["unknown_critical"] = encode(s, 2, 8, before_idat=[(b"ABCD", b"x")])
    bad["short_image_data"] = encode(s, 2, 8, raw_tail=5)
    no_idat = good[:33] + _chunk(b"IEND", b"")
    bad["no_idat"] = no_idat
    zh = bytearray(zlib.compress(b"\x00" * 10))
    zh[0] = 0x79  # compression method 9
    bad["zlib_header"] = good[:33] + _chunk(b"IDAT", bytes(zh)) + _chunk(b"IEND", b"")
    corrupt = zlib.compress(bytes(200))
    corrupt = corrupt[:2] + b"\xff\xff\xff" + corrupt[5:]
    bad["corrupt_deflate"] = good[:33] + _chunk(b"IDAT", corrupt) + _chunk(b"IEND", b"")
    return bad


MALFORMED = _malformed()


@pytest.mark.parametrize("name", sorted(MALFORMED))
def test_png_malformed_refused(name):
    png = MALFORMED[name]
    with pytest.raises(op.PngError):
        op.decode_rgb(png)
    with pytest.raises(ocrhip.OcrError, match="png"):
        ocrhip.decode_png(png, out=np.zeros(7 * 6 * 3 + 64, np.uint8))


def test_png_output_too_small():
    png = encode(np.zeros((6, 7, 3), np.int64), 2, 8)
    with pytest.raises(ocrhip.OcrError, match="output buffer"):
        ocrhip.decode_png(png, out=np.zeros(7 * 6 * 3 - 1, np.uint8))


def test_png_reference_pages_match_golden():
    """Every page PNG the reference ships (2550 x 3300 RGB at 300 dpi and the other resolutions),
    decoded by the library on four threads, against Pillow's pixels."""
    if not os.path.isdir(PAGES):
        pytest.skip("the reference's data/pages is not present")
    golden = json.load(open(GOLDEN))
    names = sorted(golden)
    assert len(names) == len(glob.glob(os.path.join(PAGES, "*", "*.png")))
    pages = ocrhip.decode_pngs([os.path.join(PAGES, n) for n in names], threads=4)
    for n, rgb in zip(names, pages):
        g = golden[n]
        assert rgb.shape == (g["h"], g["w"], 3), n
        assert hashlib.sha256(rgb.tobytes()).hexdigest() == g["sha256"], n
