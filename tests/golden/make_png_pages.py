"""Writes png_pages.json: width, height and the SHA-256 of the 8-bit RGB pixels of each of the
reference's page PNGs (data/pages/*/*.png, the pages its benchmarks decode with
image::open(p)?.into_rgb8(), src/bin/ocr-bench.rs:424), decoded by Pillow, an independent PNG
decoder. The PNGs themselves stay in the reference tree; tests/test_png.py checks the library's
decoder against these hashes where that tree is present.

    python tests/golden/make_png_pages.py [/root/reference]
"""
import glob
import hashlib
import json
import os
import sys

import numpy as np
from PIL import Image

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
out = {}
for path in sorted(glob.glob(os.path.join(ref, "data", "pages", "*", "*.png"))):
    with Image.open(path) as im:
        rgb = np.asarray(im.convert("RGB"))
    name = os.path.relpath(path, os.path.join(ref, "data", "pages"))
    out[name] = {"w": int(rgb.shape[1]), "h": int(rgb.shape[0]), "sha256": hashlib.sha256(rgb.tobytes()).hexdigest()}
    print(name, out[name]["w"], out[name]["h"])
dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "png_pages.json")
with open(dst, "w") as f:
    json.dump(out, f, indent=1, sort_keys=True)
print(f"{len(out)} pages -> {dst}")
