"""The C-ABI library without a GPU: it loads, exports every entry point include/hymoe.h declares, the Python
binding covers them all, answers the host-only queries, rejects bad arguments with the documented codes,
and the C++ header compiles."""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

import hyper_amd
from hyper_amd import HyError, check, lib

ROOT = Path(__file__).resolve().parents[1]


def declared() -> set:
    text = (ROOT / "include/hymoe.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(hy_[a-z0-9_]+)\s*\(", text))


def test_exports_every_declared_symbol():
    names = declared()
    assert len(names) >= 18
    L = lib()
    for n in sorted(names):
        assert hasattr(L, n), f"libhymoe.so does not export {n}"
    assert names == set(hyper_amd.SIGNATURES), "Python signatures out of step with the header"


# block geometry of every expert type (src/gguf.cpp:43-82) and its activation partner (8 = Q8_0, 15 = Q8_K)
EXPERT_TYPES = {6: (22, 32, 8), 7: (24, 32, 8), 8: (34, 32, 8), 10: (84, 256, 15), 11: (110, 256, 15), 12: (144, 256, 15),
                13: (176, 256, 15), 14: (210, 256, 15), 16: (66, 256, 15), 17: (74, 256, 15), 18: (98, 256, 15),
                19: (50, 256, 15), 20: (18, 32, 8), 21: (110, 256, 15), 22: (82, 256, 15), 23: (136, 256, 15),
                39: (17, 32, 8)}


def test_host_queries():
    L = lib()
    assert L.hy_abi_version() == 2
    for t, (bb, be, vt) in EXPERT_TYPES.items():
        assert (L.hy_block_bytes(t), L.hy_block_elems(t), L.hy_vec_dot_type(t)) == (bb, be, vt), t
    assert L.hy_block_bytes(15) == 292 and L.hy_block_elems(15) == 256
    assert L.hy_vec_dot_type(20) == 8 and L.hy_vec_dot_type(12) == 15 and L.hy_vec_dot_type(2) == -1
    assert L.hy_q8_row_bytes(15, 2048) == 8 * 292 and L.hy_q8_row_bytes(8, 4096) == 128 * 34 and L.hy_q8_row_bytes(15, 100) == 0


def test_argument_errors_need_no_gpu():
    """Validation happens before any HIP call: the codes and messages of the reference's throw sites."""
    from hyper_amd import hy_moe_dev
    L = lib()
    p = ctypes.c_void_p(16)
    assert L.hy_moe_route(None, 129, 128, 8, p, p, None, 1, None) == hyper_amd.HY_EINVAL
    rc = L.hy_moe_route(p, 2000, 2000, 8, p, p, None, 1, None)
    assert rc == hyper_amd.HY_EBAD_SHAPE and b"too many experts" in L.hy_last_error()
    with pytest.raises(HyError):
        check(L.hy_moe_route(p, 128, 128, 200, p, p, None, 1, None))
    m = hy_moe_dev()
    m.gate = m.up = m.down = m.slot = 16
    m.tg, m.td, m.ff, m.n, m.n_expert, m.n_local = 2, 12, 768, 2048, 128, 128   # Q4_0 gate: no kernels for it
    rc = L.hy_moe_gate_up(ctypes.byref(m), p, 2048, p, 8, p, 1, None, None, None)
    assert rc == hyper_amd.HY_EUNSUPPORTED_TYPE
    m.tg, m.gate_bytes = 12, 1234                                   # wrong bytes per expert matrix
    assert L.hy_moe_gate_up(ctypes.byref(m), p, 2048, p, 8, p, 1, None, None, None) == hyper_amd.HY_EBAD_SHAPE
    assert L.hy_q8_quantize(15, p, 2048, 300, 1, p, None) == hyper_amd.HY_EBAD_SHAPE


def test_cpp_header_compiles(tmp_path):
    gxx = shutil.which("g++")
    if not gxx or not Path("/opt/rocm/include/hip/hip_runtime_api.h").exists():
        pytest.skip("g++ or the HIP headers are not installed")
    src = tmp_path / "t.cpp"
    src.write_text('#include "hymoe.hpp"\nint main() { hymoe::MoeDev m{}; (void) m; return hy_abi_version() == 2 ? 0 : 1; }\n')
    r = subprocess.run([gxx, "-std=c++17", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}",
                        "-I/opt/rocm/include", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_tile_rows_layout():
    """tile_rows puts span s of row r at ((r // 16) * nspan + s) * 16 * sb + (r % 16) * sb of each expert, and the
    bytes of every span move whole."""
    import torch
    from hyper_amd.moe import tile_rows
    E, rows, in_dim, sb = 2, 48, 1024, 144
    nspan = in_dim // 256
    raw = torch.randint(0, 256, (E, rows, nspan * sb), dtype=torch.uint8)
    t = tile_rows(raw, in_dim).reshape(E, -1)
    for e in range(E):
        for r in (0, 1, 15, 16, 31, 47):
            for s in range(nspan):
                off = ((r // 16) * nspan + s) * 16 * sb + (r % 16) * sb
                assert torch.equal(t[e, off:off + sb], raw[e, r, s * sb:(s + 1) * sb])
    with pytest.raises(ValueError):
        tile_rows(raw[:, :40], in_dim)


def _dev(tg=12, td=14, ff=768, n=2048, E=128):
    from hyper_amd import hy_moe_dev
    m = hy_moe_dev()
    m.gate = m.up = m.down = m.slot = 16
    m.tg, m.td, m.ff, m.n, m.n_expert, m.n_local = tg, td, ff, n, E, E
    m.gate_bytes = ff * (n // 256) * {12: 144, 13: 176, 14: 210}[tg]
    m.down_bytes = n * (ff // 256) * {12: 144, 13: 176, 14: 210}[td]
    return m


def test_descriptor_rows_checked_for_every_entry():
    """Every entry point that reads a hy_moe_dev checks both ff and n against the kernels' 256-row units, also the
    matrices it does not read: a gate/up-only descriptor with ff = 800 or a down-only one with n = 2100 is rejected."""
    L = lib()
    p = ctypes.c_void_p(16)
    m = _dev(ff=800)
    m.gate_bytes = 800 * 8 * 144
    assert L.hy_moe_gate_up(ctypes.byref(m), p, 2048, p, 8, p, 1, None, None, None) == hyper_amd.HY_EBAD_SHAPE
    assert b"multiples of 256" in L.hy_last_error()
    m = _dev(n=2100)
    m.down_bytes = 2100 * 3 * 210
    assert L.hy_moe_down_reduce(ctypes.byref(m), p, p, p, 8, None, None, p, 1, None) == hyper_amd.HY_EBAD_SHAPE
    assert L.hy_moe_gemm_down(ctypes.byref(m), p, 64, p, p, p, 8, p, p, None) == hyper_amd.HY_EBAD_SHAPE


def test_grouped_gemm_rejects_more_work_items_than_its_fields_hold():
    """k_gemm keeps per-class item prefixes in 16-bit fields: a launch whose item bound reaches 2^16 is refused on the
    host (ff 768 down: 4.2 M pairs stay below the 4 GB activation limit but make 65,536 + items)."""
    L = lib()
    p = ctypes.c_void_p(16)
    m = _dev()
    rc = L.hy_moe_gemm_down(ctypes.byref(m), p, 64 * 65536, p, p, p, 128, p, p, None)
    assert rc == hyper_amd.HY_EBAD_SHAPE and b"work items" in L.hy_last_error()
    rc = L.hy_moe_gemm_gate_up(ctypes.byref(m), p, 1, 64 * 65536, p, p, p, 128, p, None)
    assert rc == hyper_amd.HY_EBAD_SHAPE


def test_upload_rejects_bad_slots():
    """hy_upload_experts validates the slot table before it allocates: -1 or a local index below E, each used once."""
    from hyper_amd import hy_expert_tensors, hy_moe_dev
    import numpy as np
    L = lib()
    E, ff, n = 4, 256, 256
    gb, db = ff * 144, n * 144
    buf = np.zeros(E * max(gb, db), np.uint8)
    t = hy_expert_tensors()
    t.gate = t.up = t.down = buf.ctypes.data
    t.gb, t.db, t.E, t.tg, t.td = gb, db, E, 12, 12
    out = hy_moe_dev()
    for bad in ([0, 1, 1, 2], [0, 1, 2, 4], [0, -2, 1, 2], [0, 1, 2, 1 << 30]):
        sl = np.array(bad, np.int32)
        rc = L.hy_upload_experts(ctypes.byref(t), sl.ctypes.data_as(ctypes.c_void_p), ff, n, 0.0, ctypes.byref(out))
        assert rc == hyper_amd.HY_EINVAL, bad
        assert b"slot" in L.hy_last_error()


def test_noalloc_decode_rejects_what_its_scratch_cannot_hold():
    """hy_moe_decode_noalloc refuses, before any device call, a step whose intermediates exceed its 1 MiB scratch array
    (64 rows of a d_model 7168, top-6, ff 2048 layer need several MiB)."""
    L = lib()
    p = ctypes.c_void_p(256)
    m = _dev(tg=12, td=12, ff=2048, n=7168, E=384)
    assert L.hy_moe_decode_ws_bytes(ctypes.byref(m), 384, 6, None, 64) > (1 << 20)
    rc = L.hy_moe_decode_noalloc(ctypes.byref(m), p, 384, p, 7168, None, 0, 6, None, p, 0, 64, None)
    assert rc == hyper_amd.HY_EBAD_SHAPE and b"scratch" in L.hy_last_error()


def test_descriptor_weights_16_byte_aligned():
    """The kernels read weight bytes in 16-byte pieces from tiles that start 16-byte aligned: a gate, up or down
    matrix that does not start on 16 bytes is rejected before any device work."""
    L = lib()
    p = ctypes.c_void_p(16)
    for field in ("gate", "up", "down"):
        m = _dev()
        setattr(m, field, 16 + 2)
        assert L.hy_moe_gate_up(ctypes.byref(m), p, 2048, p, 8, p, 1, None, None, None) == hyper_amd.HY_EBAD_SHAPE
        assert b"16-byte aligned" in L.hy_last_error()


def test_type_ids_agree_across_header_python_and_oracle():
    """include/hymoe.h's HY_* type ids, hyper_amd.formats.GType and the oracle's ids name the same GGUF type ids
    (src/gguf.h:13-18), and every expert type there has the block geometry above."""
    import oracle as orc
    from hyper_amd.formats import GType, block_bytes, block_elems, vec_dot_type
    text = (ROOT / "include/hymoe.h").read_text()
    header = {m.group(1): int(m.group(2)) for m in re.finditer(r"\bHY_([A-Z0-9_]+)\s*=\s*(\d+)", text)
              if not m.group(1).startswith("E")}
    assert {k: v for k, v in header.items() if k not in ("OK",)} == {t.name: int(t) for t in GType}
    for t in GType:
        assert getattr(orc, t.name) == int(t)
        if int(t) in EXPERT_TYPES:
            bb, be, vt = EXPERT_TYPES[int(t)]
            assert (block_bytes(t), block_elems(t), int(vec_dot_type(t))) == (bb, be, vt), t.name
            assert orc.BLOCK_BYTES[int(t)] == bb and orc.block_elems(t) == be and orc.vec_dot_type(t) == vt, t.name
    assert set(EXPERT_TYPES) == {int(t) for t in GType} - {15}


def test_moe_dev_layout_matches_c(tmp_path):
    """The ctypes hy_moe_dev has the C struct's size and field offsets (n_local included)."""
    from hyper_amd import hy_moe_dev
    gxx = shutil.which("g++")
    if not gxx or not Path("/opt/rocm/include/hip/hip_runtime_api.h").exists():
        pytest.skip("g++ or the HIP headers are not installed")
    fields = [f for f, _ in hy_moe_dev._fields_]
    src = tmp_path / "lay.cpp"
    src.write_text('#include "hymoe.h"\n#include <cstddef>\n#include <cstdio>\nint main() {\n'
                   '  std::printf("%zu", sizeof(hy_moe_dev));\n'
                   + "".join(f'  std::printf(" %zu", offsetof(hy_moe_dev, {f}));\n' for f in fields) + "}\n")
    exe = tmp_path / "lay"
    r = subprocess.run([gxx, "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", "-I/opt/rocm/include",
                        str(src), "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(hy_moe_dev)] + [getattr(hy_moe_dev, f).offset for f in fields]
    assert got == want


def test_n_local_is_required():
    """A descriptor without n_local (0) is refused before any launch: every slot entry is bounded by it."""
    m = _dev()
    m.n_local = 0
    p = ctypes.c_void_p(16)
    L = lib()
    assert L.hy_moe_gate_up(ctypes.byref(m), p, 2048, p, 8, p, 1, None, None, None) == hyper_amd.HY_EINVAL
    assert b"n_local" in L.hy_last_error()
    assert L.hy_moe_order(ctypes.byref(m), p, 8, 128, p, p, None, p) == hyper_amd.HY_EINVAL
    assert L.hy_moe_down_reduce(ctypes.byref(m), p, p, p, 8, None, None, p, 1, None) == hyper_amd.HY_EINVAL
