"""GGUF container reader and writer of libmoldq, on the host (no GPU): byte
identity with an independent restatement of the layout (tests/gguf_ref.py),
metadata of every value type read back, the embedding patch of
ensure_gguf_embeddings (crates/mold-inference/src/flux/pipeline.rs:488-547), and
the oracle's FP8 E4M3 decoding pinned against torch's float8_e4m3fn."""
import numpy as np
import pytest

import mold_amd
from mold_amd import GgmlDType, gguf
from oracle import oracle as O

from . import gguf_ref as R


def _tensors(rng):
    out = []
    for i, t in enumerate((O.Q4_K, O.Q8_0, O.Q6_K)):
        n, k = 3 + i, 256 * (i + 1)
        out.append((f"blk.{i}.weight", t, (n, k), rng.integers(0, 256, n * O.row_bytes(t, k), dtype=np.uint8)))
    out.append(("norm.scale", O.F32, (7,), np.arange(7, dtype=np.float32).view(np.uint8)))
    out.append(("emb", 30, (2, 5), rng.integers(0, 256, 20, dtype=np.uint8)))        # BF16
    out.append(("half", O.F16, (3, 1, 4), rng.integers(0, 256, 24, dtype=np.uint8)))
    return out


META = [("general.architecture", 8, "flux"), ("u8", 0, 200), ("i8", 1, -7), ("u16", 2, 65000), ("i16", 3, -30000),
        ("u32", 4, 4000000000), ("i32", 5, -2000000000), ("f32", 6, 1.5), ("bool", 7, True),
        ("u64", 10, 2 ** 63 + 5), ("i64", 11, -2 ** 62), ("f64", 12, -0.125),
        ("arr.i32", 9, [1, -2, 3], 5), ("arr.f32", 9, [0.5, 2.0], 6), ("arr.str", 9, ["a", "", "ccc"], 8),
        ("arr.empty", 9, [], 4), ("unicode", 8, "größe")]


@pytest.mark.parametrize("align", [32, 64])
def test_writer_bytes_match_restatement_and_read_back(tmp_path, align):
    rng = np.random.default_rng(align)
    tensors = _tensors(rng)
    meta = ([("general.alignment", 4, align)] if align != 32 else []) + META
    ref_p, lib_p = str(tmp_path / "ref.gguf"), str(tmp_path / "lib.gguf")
    R.write(ref_p, meta, tensors, alignment=align)
    w = gguf.Writer(lib_p, alignment=align)
    for kv in META:
        key, vt, v = kv[0], kv[1], kv[2]
        w.kv(key, v, type=(kv[3] if vt == 9 else vt) if vt != 8 else None)
    for name, t, shape, raw in tensors:
        w.add_tensor(name, GgmlDType(t), shape, raw)
    w.finish()
    w.close()
    assert open(lib_p, "rb").read() == open(ref_p, "rb").read()
    c = gguf.Content.read(lib_p)
    assert c.version == 3
    for kv in META:
        key, vt, v = kv[0], kv[1], kv[2]
        got = c.metadata[key]
        if vt == 6:
            assert got == np.float32(v)
        elif vt == 9 and kv[3] == 6:
            assert got == [float(np.float32(e)) for e in v]
        else:
            assert got == v, key
        assert c.metadata_types[key] == (vt, kv[3] if vt == 9 else vt)
    for name, t, shape, raw in tensors:
        info = c.tensor_infos[name]
        assert info.dtype == GgmlDType(t) and info.shape == tuple(shape) and info.offset % align == 0
        assert np.array_equal(c.tensor_bytes(name), raw)
    c.close()


def test_reader_keeps_nested_array_shape(tmp_path):
    p = str(tmp_path / "n.gguf")
    R.write(p, [("nested", 9, [(4, [1, 2]), (4, [3])], 9), ("after", 4, 9)],
            [("w", O.Q8_0, (1, 32), np.zeros(34, np.uint8))])
    c = gguf.Content.read(p)
    assert c.metadata_types["nested"] == (9, 9) and c.metadata["nested"] is None
    assert c.metadata["after"] == 9
    assert np.array_equal(c.tensor_bytes("w"), np.zeros(34, np.uint8))
    c.close()


def test_writer_rejects_bad_input(tmp_path):
    w = gguf.Writer(str(tmp_path / "x.gguf"))
    w.kv("a", 1)
    with pytest.raises(mold_amd.MoldqError):
        w.kv("a", 2)
    w.add_tensor("t", GgmlDType.Q8_0, (1, 32), np.zeros(34, np.uint8))
    with pytest.raises(mold_amd.MoldqError):
        w.add_tensor("t", GgmlDType.Q8_0, (1, 32), np.zeros(34, np.uint8))
    with pytest.raises(mold_amd.MoldqError):
        w.add_tensor("u", GgmlDType.Q8_0, (1, 32), np.zeros(33, np.uint8))
    with pytest.raises(mold_amd.MoldqError):
        w.add_tensor("v", GgmlDType.Q4_K, (1, 100), np.zeros(144, np.uint8))
    w.finish()
    with pytest.raises(mold_amd.MoldqError):
        w.finish()
    w.close()
    assert sorted(p.name for p in tmp_path.iterdir()) == ["x.gguf"]   # no temp file left


def _embed_gguf(path, names, rng, extra=()):
    ts = [(n, O.Q8_0 if n.endswith("weight") else O.F32, (2, 64) if n.endswith("weight") else (16,),
           rng.integers(0, 256, 2 * 68 if n.endswith("weight") else 64, dtype=np.uint8)) for n in names]
    ts += list(extra)
    R.write(path, [], ts)
    return {t[0]: t for t in ts}


@pytest.mark.parametrize("is_schnell", [True, False])
def test_patch_embeddings(tmp_path, is_schnell):
    rng = np.random.default_rng(3)
    blocks = [(f"double_blocks.{i}.img_mlp.0.weight", O.Q4_K, (2, 256), rng.integers(0, 256, 288, dtype=np.uint8))
              for i in range(3)]
    src = str(tmp_path / "city96.gguf")
    R.write(src, [("general.architecture", 8, "flux")], blocks)
    ref = str(tmp_path / "ref.gguf")
    ref_t = _embed_gguf(ref, gguf.FLUX_EMBEDDING_TENSORS + gguf.FLUX_GUIDANCE_EMBEDDING_TENSORS, rng)
    assert not gguf.has_embeddings(src) and gguf.has_embeddings(ref) and gguf.has_guidance(ref)
    dst = str(tmp_path / "patched.gguf")
    n = gguf.patch_embeddings(src, ref, dst, is_schnell)
    needed = gguf.FLUX_EMBEDDING_TENSORS + ([] if is_schnell else gguf.FLUX_GUIDANCE_EMBEDDING_TENSORS)
    assert n == len(needed)
    c = gguf.Content.read(dst)
    assert list(c.tensor_infos) == [b[0] for b in blocks] + needed
    assert c.metadata == {}
    for name, t, shape, raw in blocks:
        assert np.array_equal(c.tensor_bytes(name), raw) and c.tensor_infos[name].shape == shape
    for name in needed:
        assert np.array_equal(c.tensor_bytes(name), ref_t[name][3])
        assert c.tensor_infos[name].shape == ref_t[name][2]
    c.close()
    # a reference without guidance cannot patch a dev-family model
    ref2 = str(tmp_path / "ref_schnell.gguf")
    _embed_gguf(ref2, gguf.FLUX_EMBEDDING_TENSORS, rng)
    if is_schnell:
        assert gguf.patch_embeddings(src, ref2, str(tmp_path / "p2.gguf"), True) == len(gguf.FLUX_EMBEDDING_TENSORS)
    else:
        with pytest.raises(ValueError, match="guidance_in.in_layer.weight"):
            gguf.patch_embeddings(src, ref2, str(tmp_path / "p2.gguf"), False)


def test_oracle_e4m3_matches_torch_exhaustively():
    import torch
    b = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(b).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_to_f32(b)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert float(got[0x7E]) == 448.0 and float(got[0x01]) == 2.0 ** -9
