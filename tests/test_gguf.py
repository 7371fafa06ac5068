"""GGUF expert loading on the CPU (no GPU needed): libhymoe's reader (hy_gguf_*, replacing src/gguf.cpp:84-285 and
src/experts.cu:12-22) over files written by tests/gguf_writer.py -- every metadata kind, the tensor table and its
bytes, split models, one layer's expert tensors, and each documented failure."""
import numpy as np
import pytest
import torch

from hyper_amd import HY_EBAD_SHAPE, HY_EINVAL, HY_EUNSUPPORTED_TYPE, HyError
from hyper_amd.formats import GType, random_layer, row_bytes
from hyper_amd.gguf import GGUF, expert_layer

from .gguf_writer import ARR, BOOL, F32, F64, I8, I32, I64, STR, U8, U32, U64, write_gguf

E, D, FF = 4, 512, 256


def _layer(seed=5):
    return random_layer(GType.Q4_K, GType.Q6_K, E, FF, D, seed=seed)


def _expert_tensors(L, il=0, gate_type=None):
    """The three expert tensors of layer il in GGUF order: gate/up ne = [d, ff, E], down ne = [ff, d, E]."""
    tg = int(gate_type if gate_type is not None else L.tg)
    return [(f"blk.{il}.ffn_gate_exps.weight", tg, [D, FF, E], L.gate.numpy().tobytes()),
            (f"blk.{il}.ffn_up_exps.weight", int(L.tg), [D, FF, E], L.up.numpy().tobytes()),
            (f"blk.{il}.ffn_down_exps.weight", int(L.td), [FF, D, E], L.down.numpy().tobytes())]


KV = [("general.architecture", STR, "qwen3moe"),
      ("general.alignment", U32, 64),
      ("qwen3moe.expert_count", U32, E),
      ("qwen3moe.block_count", I32, 1),
      ("qwen3moe.rope.freq_base", F32, 1000000.0),
      ("qwen3moe.eps", F64, 1e-6),
      ("qwen3moe.use_bias", BOOL, 1),
      ("some.i8", I8, -7),
      ("some.i64", I64, -5),
      ("some.u64", U64, 1 << 40),
      ("some.int_arr", ARR, (I32, [3, -1, 7])),
      ("some.u8_arr", ARR, (U8, [255, 0])),
      ("some.float_arr", ARR, (F32, [0.5, 1.5, -2.0])),
      ("tokenizer.ggml.tokens", ARR, (STR, ["a", "bc", ""]))]


def _model(tmp_path, L, name="m.gguf", **kw):
    rng = np.random.default_rng(3)
    emb = rng.standard_normal((10, 64)).astype(np.float16)
    norm = rng.standard_normal(64).astype(np.float32)
    tensors = [("token_embd.weight", 1, [64, 10], emb.tobytes()), ("blk.0.attn_norm.weight", 0, [64], norm.tobytes())]
    tensors += _expert_tensors(L)
    p = tmp_path / name
    write_gguf(p, KV, tensors, alignment=64, **kw)
    return p, emb, norm


def test_metadata_of_every_kind(tmp_path):
    p, _, _ = _model(tmp_path, _layer())
    with GGUF(p) as g:
        assert g.arch() == "qwen3moe"
        assert g.has("qwen3moe.expert_count") and not g.has("nope")
        assert g.get_int("qwen3moe.expert_count") == E and g.get_int("qwen3moe.block_count") == 1
        assert g.get_int("some.i8") == -7 and g.get_int("some.i64") == -5 and g.get_int("some.u64") == 1 << 40
        assert g.get_int("qwen3moe.use_bias") == 1            # a bool reads as an int (src/gguf.cpp:241)
        assert g.get_int("nope", 9) == 9
        assert g.get_float("qwen3moe.rope.freq_base") == 1000000.0 and g.get_float("qwen3moe.eps") == 1e-6
        assert g.get_float("qwen3moe.expert_count") == float(E)   # an int reads as a float (src/gguf.cpp:249)
        assert g.get_str("general.architecture") == "qwen3moe"
        assert g.get_int_arr("some.int_arr") == [3, -1, 7] and g.get_int_arr("some.u8_arr") == [255, 0]
        assert g.get_int_arr("qwen3moe.expert_count") == [E]      # a scalar reads as one element
        assert g.get_float_arr("some.float_arr") == [0.5, 1.5, -2.0]
        assert g.get_float_arr("qwen3moe.rope.freq_base") == [1000000.0]
        for bad in (lambda: g.get_int("general.architecture"), lambda: g.get_str("qwen3moe.expert_count"),
                    lambda: g.get_int("missing.key"), lambda: g.get_float("tokenizer.ggml.tokens"),
                    lambda: g.get_int_arr("some.float_arr")):
            with pytest.raises(HyError) as e:
                bad()
            assert e.value.code == HY_EINVAL


def test_tensor_table_and_bytes(tmp_path):
    L = _layer()
    p, emb, norm = _model(tmp_path, L)
    with GGUF(p) as g:
        ts = g.tensors()
        assert list(ts) == ["token_embd.weight", "blk.0.attn_norm.weight", "blk.0.ffn_gate_exps.weight",
                            "blk.0.ffn_up_exps.weight", "blk.0.ffn_down_exps.weight"]
        t = ts["token_embd.weight"]
        assert (t.type, t.ne, t.nbytes) == (1, (64, 10), emb.nbytes)
        assert np.array_equal(t.data().view(np.float16).reshape(10, 64), emb)
        assert np.array_equal(g.need("blk.0.attn_norm.weight").data().view(np.float32), norm)
        gt = ts["blk.0.ffn_gate_exps.weight"]
        assert (gt.type, gt.ne, gt.nbytes) == (int(GType.Q4_K), (D, FF, E), E * FF * row_bytes(GType.Q4_K, D))
        assert g.tensor("blk.1.ffn_gate_exps.weight") is None
        with pytest.raises(HyError) as e:
            g.need("blk.1.ffn_gate_exps.weight")
        assert e.value.code == HY_EINVAL
        # data offsets honour general.alignment (64) from an aligned start of the tensor data
        assert all(x.ptr % 64 == 0 for x in ts.values())


def test_expert_tensors_and_layer(tmp_path):
    L = _layer()
    p, _, _ = _model(tmp_path, L)
    with GGUF(p) as g:
        t = g.expert_tensors(0, E)
        assert (t.E, t.tg, t.td) == (E, int(GType.Q4_K), int(GType.Q6_K))
        assert t.gb == L.gate_bytes and t.db == L.down_bytes
        assert t.gate == g.need("blk.0.ffn_gate_exps.weight").ptr and t.down == g.need("blk.0.ffn_down_exps.weight").ptr
        X = expert_layer(g, 0)
        assert (X.tg, X.td, X.E, X.ff, X.n) == (L.tg, L.td, E, FF, D)
        for a, b in ((X.gate, L.gate), (X.up, L.up), (X.down, L.down)):
            assert a.shape == b.shape and torch.equal(a, b)
        with pytest.raises(HyError) as e:   # the gate tensor (294,912 bytes) does not split into 5 experts
            g.expert_tensors(0, 5)
        assert e.value.code == HY_EBAD_SHAPE
        with pytest.raises(HyError) as e:   # no layer 1
            g.expert_tensors(1, E)
        assert e.value.code == HY_EINVAL


def test_split_model(tmp_path):
    """<name>-00001-of-00002.gguf maps both shards; metadata from the first, tensors from either."""
    L = _layer(9)
    et = _expert_tensors(L)
    write_gguf(tmp_path / "m-00001-of-00002.gguf", KV, et[:2], alignment=64)
    write_gguf(tmp_path / "m-00002-of-00002.gguf", [("general.architecture", STR, "other"), ("split.no", U32, 1)],
               et[2:], alignment=32)
    with GGUF(tmp_path / "m-00001-of-00002.gguf") as g:
        assert g.arch() == "qwen3moe" and not g.has("split.no")
        assert len(g.tensors()) == 3
        X = expert_layer(g, 0)
        assert torch.equal(X.down, L.down) and torch.equal(X.gate, L.gate)


def test_version_2_is_read(tmp_path):
    L = _layer()
    write_gguf(tmp_path / "v2.gguf", KV[:2], _expert_tensors(L), alignment=64, version=2)
    with GGUF(tmp_path / "v2.gguf") as g:
        assert torch.equal(expert_layer(g, 0).up, L.up)


def _open_code(path):
    with pytest.raises(HyError) as e:
        GGUF(path)
    return e.value.code


def test_open_failures(tmp_path):
    L = _layer()
    et = _expert_tensors(L)
    good = tmp_path / "good.gguf"
    write_gguf(good, KV[:2], et, alignment=64)
    raw = good.read_bytes()
    cases = {
        "missing.gguf": None,
        "magic.gguf": b"GGUX" + raw[4:],
        "v1.gguf": raw[:4] + (1).to_bytes(4, "little") + raw[8:],
        "trunc_head.gguf": raw[:60],
        "trunc_data.gguf": raw[:-1000],
    }
    for name, data in cases.items():
        if data is not None:
            (tmp_path / name).write_bytes(data)
        assert _open_code(tmp_path / name) == HY_EINVAL, name
    write_gguf(tmp_path / "dup.gguf", KV[:2], [et[0], et[0]], alignment=64)
    assert _open_code(tmp_path / "dup.gguf") == HY_EINVAL
    write_gguf(tmp_path / "noarch.gguf", [KV[1]], et, alignment=64)
    assert _open_code(tmp_path / "noarch.gguf") == HY_EINVAL
    q8k = [("x.weight", 15, [256, 2], bytes(2 * 292))]   # Q8_K: outside the reader's table (src/gguf.cpp:43-82)
    write_gguf(tmp_path / "q8k.gguf", KV[:2], q8k, alignment=64)
    assert _open_code(tmp_path / "q8k.gguf") == HY_EUNSUPPORTED_TYPE
    ragged = [("x.weight", 12, [300, 2], bytes(1000))]   # a Q4_K row of 300 values is not whole blocks
    write_gguf(tmp_path / "ragged.gguf", KV[:2], ragged, alignment=64)
    assert _open_code(tmp_path / "ragged.gguf") == HY_EINVAL


def test_gate_up_types_must_match(tmp_path):
    L = _layer()
    write_gguf(tmp_path / "mix.gguf", KV[:2], _expert_tensors(L, gate_type=GType.Q5_K)[:0] +
               [("blk.0.ffn_gate_exps.weight", int(GType.Q5_K), [D, FF, E], bytes(E * FF * row_bytes(GType.Q5_K, D)))] +
               _expert_tensors(L)[1:], alignment=64)
    with GGUF(tmp_path / "mix.gguf") as g:
        with pytest.raises(HyError) as e:
            g.expert_tensors(0, E)
        assert e.value.code == HY_EBAD_SHAPE


def test_corrupted_files_fail_cleanly(tmp_path):
    """Truncations and byte flips anywhere in a file: the open either succeeds or returns an error, never crashes,
    and whatever it accepts stays inside the mapping."""
    L = _layer()
    good = tmp_path / "good.gguf"
    write_gguf(good, KV, _expert_tensors(L), alignment=64)
    raw = bytearray(good.read_bytes())
    rng = np.random.default_rng(11)
    head = len(raw) - len(L.gate.numpy().tobytes()) * 2 - len(L.down.numpy().tobytes())
    p = tmp_path / "bad.gguf"
    for i in range(300):
        b = bytearray(raw)
        if i % 3 == 0:
            b = b[: int(rng.integers(1, len(b)))]
        else:
            for _ in range(int(rng.integers(1, 4))):
                pos = int(rng.integers(0, head))
                b[pos] = int(rng.integers(0, 256))
        p.write_bytes(bytes(b))
        try:
            with GGUF(p) as g:
                for t in g.tensors().values():
                    if t.nbytes:
                        int(t.data()[0]) + int(t.data()[-1])   # both ends of every accepted view are readable
        except HyError as e:
            assert e.code in (HY_EINVAL, HY_EUNSUPPORTED_TYPE)
