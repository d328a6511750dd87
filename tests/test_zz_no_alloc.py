"""The allocation-free word boxes (ocr_word_rects_gpu_noalloc, labelling in the library's fixed
device array) against ocr_word_rects_gpu (pooled buffers): the same rectangles, bit for bit, on
consecutive calls with smaller and larger masks (the array keeps the previous call's contents),
on a mask past the array's run capacity (labelled on the host), and a clear error for masks
larger than the array."""
import numpy as np
import pytest

import ocrhip
from ocrhip import synth

pytestmark = pytest.mark.gpu


def _pack(mask: np.ndarray) -> np.ndarray:
    h, w = mask.shape
    padded = np.zeros((h, (w + 31) // 32 * 32), bool)
    padded[:, :w] = mask
    return np.packbits(padded, axis=1, bitorder="little").view(np.uint32).copy()


def _same(ctx, bits, w, what):
    print(f"noalloc word rects: {what} ({bits.shape[0]} x {w})", flush=True)
    want = ocrhip.word_rects_gpu(ctx, bits, w)
    got = ocrhip.word_rects_gpu_noalloc(ctx, bits, w)
    assert got.shape == want.shape, what
    np.testing.assert_array_equal(got, want)
    return got


def test_noalloc_word_rects_match_pooled_entry(detector, ctx):
    page = synth.page(3)
    full = detector.detect_page(page, 0.5)
    a = _same(ctx, full, page.shape[1], "full page mask")
    assert len(a) > 100
    # The second call with a smaller input: the top part of the same page, then a small noise mask.
    b = _same(ctx, np.ascontiguousarray(full[:900]), page.shape[1], "top 900 rows")
    assert 0 < len(b) < len(a)
    rng = np.random.Generator(np.random.PCG64(5))
    _same(ctx, _pack(rng.random((97, 333)) < 0.45), 333, "noise")
    _same(ctx, _pack(np.zeros((8, 40), bool)), 40, "empty")
    # More runs than the array holds: the host labels it, the same rectangles.
    _same(ctx, _pack(rng.random((700, 1500)) < 0.5), 1500, "noise past the run capacity")
    # And a full page again after those.
    _same(ctx, full, page.shape[1], "full page mask again")


def test_noalloc_word_rects_allocate_nothing():
    # A context of its own, used by nothing else: its pool starts empty. The allocation-free
    # entry, called on masks of decreasing size, must leave the library's device and page-locked
    # allocation counts and the pool untouched; the pooled entry afterwards does allocate.
    ctx = ocrhip.Context(pool_mb=64)
    rng = np.random.Generator(np.random.PCG64(11))
    masks = [(_pack(rng.random((1200, 2000)) < 0.3), 2000), (_pack(rng.random((300, 700)) < 0.3), 700)]
    print("noalloc word rects: allocation counts", flush=True)
    before = ctx.memory_stats()
    for bits, w in masks:
        ocrhip.word_rects_gpu_noalloc(ctx, bits, w)
    after = ctx.memory_stats()
    assert after == before, (before, after)
    ocrhip.word_rects_gpu(ctx, *masks[1])
    pooled = ctx.memory_stats()
    assert pooled["device_allocs"] > after["device_allocs"] or pooled["pool_held"] > after["pool_held"]
    ctx.close()


def test_noalloc_word_rects_reject_oversize(ctx):
    print("noalloc word rects: oversize masks", flush=True)
    with pytest.raises(ocrhip.OcrError, match="exceed"):
        ocrhip.word_rects_gpu_noalloc(ctx, np.zeros((16385, 1), np.uint32), 32)
    with pytest.raises(ocrhip.OcrError, match="exceed"):
        ocrhip.word_rects_gpu_noalloc(ctx, np.zeros((4096, 129), np.uint32), 4128)
    # The largest accepted mask still works after the refusals.
    bits = np.zeros((4096, 128), np.uint32)
    bits[100:120, 10:20] = 0xFFFFFFFF
    _same(ctx, bits, 4096, "largest mask")
