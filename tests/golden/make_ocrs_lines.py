"""Writes ocrs_lines.npz: word masks of the reference's four 300-dpi pages and the lines ocrs
0.13.1 found on them, the fixture that pins the page layout's line grouping and reading order to
ocrs's own output (ocrs `find_text_lines`, called at src/bin/ocr-bench.rs:516).

- Pages: data/pages/A_300/Text_page_1..4.png (2550 x 3300 RGB), the pages of the reference's
  benchmark (README.md:13).
- ocrs's lines: results/texts-245k/ocrs_0..3.txt, "ocrs 0.13.1 on the CPU as shipped"
  (results/README.md), one recognised line a line of the file. The files end without a newline,
  so they hold 43, 42, 42 and 17 lines. Only each line's character count is kept (`chars_k`):
  text from ocrs's real recogniser is not reproducible with the random-init models here, but a
  line's length tracks the width of the page line it came from.
- Word masks (`bits_k`, h rows of ceil(w / 32) words, bit x % 32 of word x / 32): the ocrs
  detector is a trained network that cannot be fetched here, so a stand-in marks word blobs:
  ink where 299 R + 587 G + 114 B < 128000 (grey below 128), dilated by a 9-row x 13-column box,
  which closes the gaps inside words (1-12 px at 300 dpi, punctuation included) and keeps the
  gaps between words (13 px and more). word_mask() is that rule; tests/test_ocrs_lines.py applies
  it to ocr_png_decode's pixels and checks it gives these masks where the reference is present.

    python tests/golden/make_ocrs_lines.py [/root/reference]
"""
import os
import sys

import numpy as np

PAGES = 4


def word_mask(rgb: np.ndarray) -> np.ndarray:
    """The stand-in detector: bit-packed word blobs of an h x w x 3 u8 page."""
    from scipy import ndimage as ndi

    rgb = rgb.astype(np.int32)
    ink = (299 * rgb[..., 0] + 587 * rgb[..., 1] + 114 * rgb[..., 2]) < 128000
    mask = ndi.binary_dilation(ink, structure=np.ones((9, 13), bool))
    h, w = mask.shape
    padded = np.zeros((h, (w + 31) // 32 * 32), bool)
    padded[:, :w] = mask
    return np.packbits(padded, axis=1, bitorder="little").view(np.uint32).copy()


def ocrs_line_lengths(ref: str, k: int) -> np.ndarray:
    with open(os.path.join(ref, "results", "texts-245k", f"ocrs_{k}.txt"), encoding="utf-8") as f:
        return np.array([len(line) for line in f.read().split("\n")], np.int32)


def main():
    from PIL import Image

    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    out = {}
    for k in range(PAGES):
        path = os.path.join(ref, "data", "pages", "A_300", f"Text_page_{k + 1}.png")
        with Image.open(path) as im:
            rgb = np.asarray(im.convert("RGB"))
        out[f"bits_{k}"] = word_mask(rgb)
        out[f"w_{k}"] = np.int32(rgb.shape[1])
        out[f"chars_{k}"] = ocrs_line_lengths(ref, k)
        print(f"page {k + 1}: {rgb.shape[1]} x {rgb.shape[0]}, {len(out[f'chars_{k}'])} ocrs lines")
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ocrs_lines.npz")
    np.savez_compressed(dst, **out)
    print(f"-> {dst} ({os.path.getsize(dst)} bytes)")


if __name__ == "__main__":
    main()
