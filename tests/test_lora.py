"""mold's GGUF LoRA path, host side: the diffusers -> candle key mapping and
fused-slice rows against the reference's own unit tests
(crates/mold-inference/src/flux/lora.rs:905-1073), and the oracle's merge
order pinned by exact cases and an f64 bound."""
import numpy as np
import pytest

from mold_amd.lora import LoraTarget, fused_slice_range, map_lora_key
from oracle import oracle as O


def test_map_double_block_qkv():
    for comp, layer in enumerate(("attn.to_q", "attn.to_k", "attn.to_v")):
        t = map_lora_key(f"transformer.transformer_blocks.5.{layer}")
        assert t == LoraTarget("double_blocks.5.img_attn.qkv.weight", comp, 3)
    assert map_lora_key("transformer.transformer_blocks.0.attn.add_q_proj") == \
        LoraTarget("double_blocks.0.txt_attn.qkv.weight", 0, 3)


def test_map_double_block_direct():
    cases = {
        "transformer.transformer_blocks.3.attn.to_out.0": "double_blocks.3.img_attn.proj.weight",
        "transformer.transformer_blocks.3.attn.to_add_out": "double_blocks.3.txt_attn.proj.weight",
        "transformer.transformer_blocks.3.ff.net.0.proj": "double_blocks.3.img_mlp.0.weight",
        "transformer.transformer_blocks.3.ff.net.2": "double_blocks.3.img_mlp.2.weight",
        "transformer.transformer_blocks.3.ff_context.net.0.proj": "double_blocks.3.txt_mlp.0.weight",
        "transformer.transformer_blocks.3.ff_context.net.2": "double_blocks.3.txt_mlp.2.weight",
        "transformer.transformer_blocks.3.norm1.linear": "double_blocks.3.img_mod.lin.weight",
        "transformer.transformer_blocks.3.norm1_context.linear": "double_blocks.3.txt_mod.lin.weight",
    }
    for k, v in cases.items():
        assert map_lora_key(k) == LoraTarget(v), k


def test_map_single_block():
    assert map_lora_key("transformer.single_transformer_blocks.7.attn.to_q") == \
        LoraTarget("single_blocks.7.linear1.weight", 0, 0)
    assert map_lora_key("transformer.single_transformer_blocks.7.proj_mlp").component == 3
    assert map_lora_key("transformer.single_transformer_blocks.7.proj_out") == LoraTarget("single_blocks.7.linear2.weight")
    assert map_lora_key("transformer.single_transformer_blocks.7.norm.linear") == \
        LoraTarget("single_blocks.7.modulation.lin.weight")
    # keys without the "transformer." prefix map the same way
    assert map_lora_key("single_transformer_blocks.7.proj_out") == LoraTarget("single_blocks.7.linear2.weight")


def test_map_unknown_key_returns_none():
    assert map_lora_key("totally.unknown.key") is None
    assert map_lora_key("transformer.transformer_blocks.0.unknown_layer") is None
    assert map_lora_key("transformer.transformer_blocks.x.attn.to_q") is None


def test_fused_slice_range_reference_cases():
    assert fused_slice_range(9216, 3072, 0, 3) == (0, 3072)
    assert fused_slice_range(9216, 3072, 1, 3) == (3072, 3072)
    assert fused_slice_range(9216, 3072, 2, 3) == (6144, 3072)
    assert fused_slice_range(21504, 3072, 0, 0) == (0, 3072)
    assert fused_slice_range(21504, 3072, 1, 0) == (3072, 3072)
    assert fused_slice_range(21504, 3072, 2, 0) == (6144, 3072)
    assert fused_slice_range(21504, 12288, 3, 0) == (9216, 12288)


def test_oracle_lora_apply_exact_on_integers():
    """Small integers: every product and partial sum is exact, so any order gives w + b.a."""
    rng = np.random.default_rng(0)
    w = rng.integers(-50, 50, (9, 70)).astype(np.float32)
    b = rng.integers(-8, 8, (9, 13)).astype(np.float32)
    a = rng.integers(-8, 8, (13, 70)).astype(np.float32)
    got = O.lora_apply(w, b, a, 1.0)
    assert np.array_equal(got, w + (b.astype(np.int64) @ a.astype(np.int64)).astype(np.float32))


def test_oracle_lora_apply_rank1_rounding():
    """Rank 1: d = round(b*a), then round(d*scale), then round(w + that), each in f32."""
    rng = np.random.default_rng(1)
    w = rng.standard_normal((5, 33)).astype(np.float32)
    b = rng.standard_normal((5, 1)).astype(np.float32)
    a = rng.standard_normal((1, 33)).astype(np.float32)
    s = np.float32(0.37)
    want = w + (b * a) * s          # numpy float32: one rounding per operation
    assert np.array_equal(O.lora_apply(w, b, a, float(s)), want)


def test_oracle_lora_apply_f64_bound():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((17, 100)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((17, 48)) * 0.1).astype(np.float32)
    a = (rng.standard_normal((48, 100)) * 0.1).astype(np.float32)
    got = O.lora_apply(w, b, a, 0.75).astype(np.float64)
    ref = w.astype(np.float64) + 0.75 * (b.astype(np.float64) @ a.astype(np.float64))
    bound = 4 * 2.0 ** -24 * (np.abs(w) + 0.75 * (np.abs(b) @ np.abs(a)) * 48)
    assert np.all(np.abs(got - ref) <= bound)


def test_adapter_alpha_only_from_rank0_f32(tmp_path):
    """LoraAdapter::load keeps `<layer>.alpha` only when `to_scalar::<f32>()`
    succeeds (lora.rs:77-79), i.e. for a rank-0 F32 tensor; a bf16 / f16 alpha or
    a shape-[1] alpha is dropped, so those layers use the plain scale."""
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file
    from mold_amd.lora import LoraAdapter, build_patches
    st = {}
    cases = {"f32_rank0": (torch.tensor(8.0), 8.0), "bf16_rank0": (torch.tensor(8.0, dtype=torch.bfloat16), None),
             "f16_rank0": (torch.tensor(8.0, dtype=torch.float16), None), "f32_shape1": (torch.tensor([8.0]), None)}
    for i, (nm, (alpha, _)) in enumerate(cases.items()):
        key = f"transformer.single_transformer_blocks.{i}.proj_out"
        st[f"{key}.lora_A.weight"] = torch.ones((4, 16))
        st[f"{key}.lora_B.weight"] = torch.ones((16, 4))
        st[f"{key}.alpha"] = alpha
    path = tmp_path / "lora.safetensors"
    save_file(st, str(path))
    ad = LoraAdapter.load(str(path))
    for i, (nm, (_, want)) in enumerate(cases.items()):
        layer = ad.layers[f"transformer.single_transformer_blocks.{i}.proj_out"]
        assert layer.alpha == want, nm
    patches, skipped = build_patches(ad, 0.5)
    assert skipped == 0
    effs = {p.target.candle_key: p.effective_scale for pl in patches.values() for p in pl}
    assert effs["single_blocks.0.linear2.weight"] == 0.5 * 8.0 / 4     # scale * alpha / rank
    for i in (1, 2, 3):
        assert effs[f"single_blocks.{i}.linear2.weight"] == 0.5       # alpha dropped
