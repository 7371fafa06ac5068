"""Write tests/golden/reference_tables.json: SHA-256 digests of the codebooks the reference carries, so the
tests can check this repository's copies without reading the reference at run time.

  iq2xs_grid:  src/iq_grids.h:80-209 (g_iq2xs_grid, 512 x u64, little-endian bytes)
  iq2xxs_grid: src/iq_grids.h:14-79  (g_iq2xxs_grid, 256 x u64, little-endian bytes)
  iq2s_grid:  src/iq_grids.h:210-467 (g_iq2s_grid, 1024 x u64, little-endian bytes)
  iq1s_grid:  src/iq_grids.h:504-1017 (g_iq1s_grid, 2048 x u64, little-endian bytes)
  iq3xxs_grid: src/iq_grids.h:468-503 (g_iq3xxs_grid, 256 x u32, little-endian bytes)
  iq3s_grid:  src/kernels4.cu:480-545 (g_iq3s_grid, 512 x u32, little-endian bytes)
  ksigns:     src/iq_grids.h:4-13   (g_ksigns_iq2xs, 128 bytes)
  iq4nl:      src/kernels4.cu:546   (g_iq4nl, 16 x int8)

Run in a checkout with the reference beside it:  python tests/golden/make_reference_tables.py [/root/reference]
"""
import hashlib
import json
import re
import sys
from pathlib import Path

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")


def array(text, name):
    m = re.search(name + r"\[\d+\]\s*=\s*\{(.*?)\};", text, re.S)
    return [int(v, 0) for v in re.findall(r"-?0x[0-9a-fA-F]+|-?\d+", m.group(1))]


grids = (ref / "src/iq_grids.h").read_text()
k4 = (ref / "src/kernels4.cu").read_text()
grid = array(grids, "g_iq2xs_grid")
grid2 = array(grids, "g_iq2xxs_grid")
grid3 = array(grids, "g_iq3xxs_grid")
grid2s = array(grids, "g_iq2s_grid")
grid1s = array(grids, "g_iq1s_grid")
grid3s = array(k4, "g_iq3s_grid")
ks = array(grids, "g_ksigns_iq2xs")
kv = array(k4, "g_iq4nl")
out = {
    "iq2xs_grid_sha256": hashlib.sha256(b"".join(v.to_bytes(8, "little") for v in grid)).hexdigest(),
    "iq2xxs_grid_sha256": hashlib.sha256(b"".join(v.to_bytes(8, "little") for v in grid2)).hexdigest(),
    "iq3xxs_grid_sha256": hashlib.sha256(b"".join(v.to_bytes(4, "little") for v in grid3)).hexdigest(),
    "iq2s_grid_sha256": hashlib.sha256(b"".join(v.to_bytes(8, "little") for v in grid2s)).hexdigest(),
    "iq1s_grid_sha256": hashlib.sha256(b"".join(v.to_bytes(8, "little") for v in grid1s)).hexdigest(),
    "iq3s_grid_sha256": hashlib.sha256(b"".join(v.to_bytes(4, "little") for v in grid3s)).hexdigest(),
    "ksigns_sha256": hashlib.sha256(bytes(ks)).hexdigest(),
    "iq4nl_sha256": hashlib.sha256(bytes(v & 0xFF for v in kv)).hexdigest(),
    "sizes": {"iq2xs_grid": len(grid), "iq2xxs_grid": len(grid2), "iq3xxs_grid": len(grid3), "iq3s_grid": len(grid3s), "iq2s_grid": len(grid2s), "iq1s_grid": len(grid1s), "ksigns": len(ks), "iq4nl": len(kv)},
}
(Path(__file__).resolve().parent / "reference_tables.json").write_text(json.dumps(out, indent=1) + "\n")
print(out)
