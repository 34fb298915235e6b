"""Writes tests/golden/ssim_window.json: the 11 SSIM window weights tabulated
in the reference (core/metal/msplat_metal.metal, SSIM_GAUSS_KERNEL), read as
text from the reference checkout.  Run in the build container:

    python tests/golden/extract_ssim_window.py /root/reference
"""
import json
import re
import sys
from pathlib import Path

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
src = (ref / "core/metal/msplat_metal.metal").read_text()
lines = src.splitlines()
start = next(i for i, l in enumerate(lines) if "SSIM_GAUSS_KERNEL[11]" in l)
block = "\n".join(lines[start:start + 14])
vals = [float(v) for v in re.findall(r"([0-9]+\.[0-9]+)f", block)][:11]
assert len(vals) == 11
out = Path(__file__).resolve().parent / "ssim_window.json"
out.write_text(json.dumps({"source": f"core/metal/msplat_metal.metal:{start + 1}-{start + 13}",
                           "weights": vals}, indent=1) + "\n")
print(out, vals)
