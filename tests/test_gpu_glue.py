"""GPU tests of libmoldq's fused block glue (mq_adaln_modulate, mq_qk_norm_rope,
mq_gelu_tanh_bf16, mq_attn_pad_correct) against torch restatements of the ops they
replace:
  modulate   LayerNorm(eps 1e-6, no affine) * (1 + scale) + shift, to bf16
             (crates/mold-inference/src/flux/offload.rs:75-78, 283-286)
  qk norm    x / sqrt(mean(x^2) + eps) * w for q and k per head (offload.rs:160-167, 188-201)
  RoPE       pair (2i, 2i+1) rotated by angle i: (c x0 - s x1, s x0 + c x1) (offload.rs:56-66)
  pad fix    o / (1 - n exp(-lse)) per (row, head) of an attention over n zero keys
The kernels compute in f32 and round once to bf16, so every output must lie within
one bf16 ulp of the f64 value (half an ulp of rounding plus f32 noise), and v, a
plain bf16 conversion, must equal torch's conversion bit for bit.  The padded
attention's correction repeats torch's f32 op sequence (exp, multiply, subtract,
reciprocal, multiply, round), so it must equal that sequence bit for bit.
"""
import numpy as np
import pytest
import torch

import mold_amd
from mold_amd import fused as FU
from mold_amd._lib import MoldqError

pytestmark = pytest.mark.gpu


def _within_one_ulp(out_bf16, ref64):
    out = out_bf16.double().cpu()
    ref = ref64.cpu()
    ulp = torch.clamp(ref.abs(), min=1e-30) * 2.0 ** -7
    return bool(((out - ref).abs() <= ulp + 1e-5).all())


@pytest.mark.parametrize("rows,cols,ld", [(1, 256, 256), (37, 3072, 3072), (300, 1024, 1280), (5, 8192, 8192)])
def test_adaln_modulate_matches_reference(rows, cols, ld):
    print(f"[case] adaln rows={rows} cols={cols} ld={ld}", flush=True)
    mold_amd.load()
    g = torch.Generator().manual_seed(rows + cols)
    xb = (torch.randn((rows, ld), generator=g) * 3 + 0.5).cuda()
    x = xb[:, :cols]
    shift = torch.randn((1, cols), generator=g).cuda()
    scale = (torch.randn((1, cols), generator=g) * 0.1).cuda()
    out = FU.adaln_modulate(x, shift, scale)
    torch.cuda.synchronize()
    xd = x.double().cpu()
    mu = xd.mean(-1, keepdim=True)
    ref = (xd - mu) / torch.sqrt(((xd - mu) ** 2).mean(-1, keepdim=True) + 1e-6)
    ref = ref * (1 + scale.double().cpu()) + shift.double().cpu()
    assert out.dtype == torch.bfloat16 and out.shape == (rows, cols)
    assert _within_one_ulp(out, ref)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,heads,extra,row_off,l_total", [(37, 3, 64, 5, 50), (512, 24, 0, 0, 512),
                                                              (64, 2, 12288 - 768, 100, 164)])
def test_qk_norm_rope_matches_reference(rows, heads, extra, row_off, l_total, dtype):
    print(f"[case] qk_norm_rope rows={rows} heads={heads} off={row_off} {dtype}", flush=True)
    mold_amd.load()
    g = torch.Generator().manual_seed(rows * heads)
    d = 128
    ld = 3 * heads * d + extra
    y = (torch.randn((rows, ld), generator=g) * 2).cuda()
    if dtype == "bf16":
        y = y.to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).cuda()
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).cuda()
    ang = torch.rand((rows, d // 2), generator=g, dtype=torch.float64) * 50
    cos, sin = torch.cos(ang).float().cuda(), torch.sin(ang).float().cuda()
    q, k, v = FU.new_heads(heads, l_total, "cuda")
    for t in (q, k, v):
        t.fill_(7.0)
    FU.qk_norm_rope(y, heads, qw, kw, cos, sin, q, k, v, row_off)
    torch.cuda.synchronize()
    yd = y.double().cpu()[:, :3 * heads * d].reshape(rows, 3, heads, d).permute(1, 2, 0, 3)  # [3, H, L, D]
    c, s = cos.double().cpu(), sin.double().cpu()

    def norm_rope(x, w):
        x = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w.double().cpu()
        x0, x1 = x[..., 0::2], x[..., 1::2]
        return torch.stack([c * x0 - s * x1, s * x0 + c * x1], dim=-1).reshape(x.shape)

    sl = slice(row_off, row_off + rows)
    assert _within_one_ulp(q[:, sl], norm_rope(yd[0], qw))
    assert _within_one_ulp(k[:, sl], norm_rope(yd[1], kw))
    vref = y[:, 2 * heads * d:3 * heads * d].reshape(rows, heads, d).transpose(0, 1).float().to(torch.bfloat16)
    assert torch.equal(v[:, sl].view(torch.int16), vref.view(torch.int16))
    # rows outside the segment are untouched
    assert bool((q[:, :row_off] == 7.0).all()) and bool((q[:, row_off + rows:] == 7.0).all())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,cols,lds,ldd,off", [(37, 12288, 21504, 15360, 9216), (5, 8, 8, 12, 0)])
def test_gelu_tanh_bf16_matches_reference(rows, cols, lds, ldd, off, dtype):
    """GELU-tanh of a strided f32 block into a strided bf16 block (the FLUX single block's
    MLP half written into linear2's concatenated input): within one bf16 ulp of f64, and
    the destination's other columns untouched."""
    print(f"[case] gelu_bf16 rows={rows} cols={cols}", flush=True)
    mold_amd.load()
    g = torch.Generator().manual_seed(rows + cols)
    src = (torch.randn((rows, lds), generator=g) * 3).cuda()
    if dtype == "bf16":
        src = src.to(torch.bfloat16)
    dst = torch.full((rows, ldd), 5.0, dtype=torch.bfloat16, device="cuda")
    sv = src[:, off:off + cols]
    dv = dst[:, ldd - cols:]
    FU.gelu_tanh_bf16(sv, dv)
    torch.cuda.synchronize()
    xd = sv.double().cpu()
    ref = 0.5 * xd * (1 + torch.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)))
    assert _within_one_ulp(dv, ref)
    assert bool((dst[:, :ldd - cols] == 5.0).all())


@pytest.mark.parametrize("valid,padded", [(295, 512), (1000, 1024), (512, 512)])
def test_padded_attention_matches_reference(valid, padded):
    """attention_bf16 over joint buffers padded with zero k / v rows (the fused paths pad the
    sequence to a multiple of 256): the log-sum-exp correction removes the zero keys exactly,
    so the result matches f32 attention on the valid rows to bf16 accuracy."""
    from mold_amd.flux import attention_bf16
    print(f"[case] padded attention valid={valid} padded={padded}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(valid)
    H, D = 4, 128
    q, k, v = (torch.randn((H, padded, D), device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    k[:, valid:] = 0
    v[:, valid:] = 0
    q[:, valid:] = 3.0  # pad query rows are never read back
    out = attention_bf16(q, k, v, valid)
    qf, kf, vf = (t[:, :valid].float() for t in (q, k, v))
    ref = torch.softmax(qf @ kf.transpose(1, 2) / np.sqrt(D), dim=-1) @ vf
    ref = ref.transpose(0, 1).reshape(valid, H * D)
    assert out.shape == (valid, H * D)
    err = ((out.float() - ref).norm() / ref.norm()).item()
    assert err < 5e-3, err
    _check_out_block(attention_bf16, (q, k, v, valid), out)


def _check_out_block(attn, args, expect):
    """attn(*args, out=block) with block a strided column block of a wider bf16 buffer
    (how the single block writes attention into linear2's input): bit-identical to the
    returned tensor, the buffer's other columns untouched."""
    valid, hd = expect.shape
    buf = torch.full((valid, hd + 96), 7.0, dtype=torch.bfloat16, device="cuda")
    block = buf[:, 32:32 + hd]
    r = attn(*args, out=block)
    torch.cuda.synchronize()
    assert r.data_ptr() == block.data_ptr()
    assert torch.equal(block, expect)
    assert bool((buf[:, :32] == 7.0).all()) and bool((buf[:, 32 + hd:] == 7.0).all())


def test_batched_padded_attention_with_dropped_keys():
    """attention_bf16_batch (one launch over [B, H, L, D], the CFG batch-2 block): element 0
    with padding only, element 1 with masked keys 30 .. 63 as well (a shorter uncond
    prompt).  Each element must match f64 attention over its own kept keys, and the guard
    must hold the largest pad share of both."""
    from mold_amd.flux import attention_bf16_batch
    B, H, D, valid, padded, lo, hi = 2, 4, 128, 700, 768, 30, 64
    print(f"[case] batched padded attention B={B} valid={valid} padded={padded} drop={lo}..{hi}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(11)
    q, k, v = (torch.randn((B, H, padded, D), device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    k[:, :, valid:] = 0
    v[:, :, valid:] = 0
    k[1, :, lo:hi] = 0
    v[1, :, lo:hi] = 0
    guard = torch.zeros((), dtype=torch.float32, device="cuda")
    out = attention_bf16_batch(q, k, v, valid=valid, guard=guard, drops=[None, (lo, hi)])
    torch.cuda.synchronize()
    assert out.shape == (B, valid, H * D)
    keep = [torch.arange(valid), torch.cat([torch.arange(lo), torch.arange(hi, valid)])]
    for b in range(B):
        qf = q[b, :, :valid].double().cpu()
        kf, vf = (t[b, :, keep[b]].double().cpu() for t in (k, v))
        ref = (torch.softmax(qf @ kf.transpose(1, 2).contiguous() / np.sqrt(D), dim=-1) @ vf)
        ref = ref.transpose(0, 1).reshape(valid, H * D)
        err = ((out[b].double().cpu() - ref).norm() / ref.norm()).item()
        assert err < 5e-3, (b, err)
    assert 0.0 < float(guard) < 0.5


def _anti_aligned(valid, padded, bad_heads, H=4, D=128, seed=7):
    """q, k, v [H, padded, D] bf16 whose heads in `bad_heads` have every valid score
    q.k/sqrt(D) <= -10 (q anti-aligned with all keys), so the zero pad keys hold
    nearly all of those rows' softmax mass."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v = (torch.randn((H, padded, D), device="cuda", generator=g) for _ in range(3))
    u = torch.randn(D, device="cuda", generator=g)
    u = u / u.norm()
    for h in bad_heads:
        k[h] = 12.0 * u + 0.05 * k[h]
        q[h] = -12.0 * u + 0.05 * q[h]
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    k[:, valid:] = 0
    v[:, valid:] = 0
    return q, k, v


def _attn_ref(q, k, v, valid):
    H, _, D = q.shape
    qf, kf, vf = (t[:, :valid].double().cpu() for t in (q, k, v))      # f64 on the host
    s = qf @ kf.transpose(1, 2).contiguous() / np.sqrt(D)
    return (torch.softmax(s, dim=-1) @ vf).transpose(0, 1).reshape(valid, H * D), s


def test_padded_attention_ill_conditioned_rows_recomputed():
    """Heads whose valid scores are all <= -10: the zero-key correction would divide by a
    valid-key share near 0, so those heads are recomputed over the valid keys."""
    from mold_amd.flux import attention_bf16
    valid, padded, bad = 700, 768, [1, 3]
    print(f"[case] anti-aligned padded attention valid={valid} padded={padded} bad heads={bad}", flush=True)
    q, k, v = _anti_aligned(valid, padded, bad)
    ref, s = _attn_ref(q, k, v, valid)
    assert float(s[bad].max()) <= -10.0
    out = attention_bf16(q, k, v, valid)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all().item()
    _check_out_block(attention_bf16, (q, k, v, valid), out)
    H, D = q.shape[0], q.shape[2]
    for h in range(H):
        o, r = out.view(valid, H, D)[:, h].double().cpu(), ref.view(valid, H, D)[:, h]
        err = ((o - r).norm() / r.norm()).item()
        assert err < 5e-3, (h, err)


def test_padded_attention_guard_and_step_rerun():
    """With a guard tensor the call only records the largest pad share; run_guarded reads
    it once and reruns the forward unpadded, which is then exact."""
    from mold_amd.flux import PAD_MIN_SHARE, attention_bf16, run_guarded
    valid, padded = 700, 768
    q, k, v = _anti_aligned(valid, padded, [0, 1, 2, 3])
    ref, _ = _attn_ref(q, k, v, valid)

    class Step:
        attn = staticmethod(attention_bf16)
        pad_attention = True
        _guard = None
        calls = []

        def fwd(self, x):
            self.calls.append(self.pad_attention)
            if self.pad_attention:
                return attention_bf16(q, k, v, valid, guard=self._guard)
            return attention_bf16(q[:, :valid], k[:, :valid], v[:, :valid])

    st = Step()
    guard = torch.zeros((), device="cuda")
    attention_bf16(q, k, v, valid, guard=guard)
    assert float(guard) > 1.0 - PAD_MIN_SHARE
    out = run_guarded(st, st.fwd, q)
    assert st.calls == [True, False] and st.pad_attention and st._guard is None
    err = ((out.double().cpu() - ref).norm() / ref.norm()).item()
    assert err < 5e-3, err


@pytest.mark.parametrize("B,H,rows,L,layout", [(1, 24, 7145, 7168, "bhld"), (2, 4, 700, 768, "blhd"),
                                                (1, 3, 5, 64, "bhld"), (2, 2, 1, 32, "blhd")])
def test_attn_pad_correct_matches_torch_sequence(B, H, rows, L, layout):
    """mq_attn_pad_correct against the torch ops it replaces in the padded attention:
    share = n_b * exp(-lse), out = bf16(o * (1 / (1 - share))) in the [rows, H*128]
    layout, guard = max(guard, max share).  o in the attention's [B, H, L, 128] view
    over head-major or row-major memory; out also as a column block of a wider buffer."""
    print(f"[case] attn_pad_correct B={B} H={H} rows={rows} L={L} {layout}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + 7 * B)
    if layout == "bhld":
        o = torch.randn((B, H, L, 128), device="cuda", generator=g).to(torch.bfloat16)
    else:
        o = torch.randn((B, L, H, 128), device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
    lse = (float(np.log(L)) + 2.0 * torch.randn((B, H, L + 5), device="cuda", generator=g))[:, :, :L]
    counts = [L - rows + 3 * b for b in range(B)]
    npad = torch.tensor(counts, dtype=torch.float32, device="cuda")
    share = npad.view(B, 1, 1) * torch.exp(-lse[:, :, :rows])
    ref = torch.empty((B, rows, H, 128), dtype=torch.bfloat16, device="cuda")
    torch.mul(o[:, :, :rows].transpose(1, 2), (1.0 / (1.0 - share)).transpose(1, 2)[..., None], out=ref)
    ref = ref.reshape(B, rows, H * 128)
    guard = torch.zeros((), dtype=torch.float32, device="cuda")
    out = FU.attn_pad_correct(o, lse, npad, rows, guard, torch.empty_like(ref))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert float(guard) == float(share.amax())
    big = torch.full((), 1e3, dtype=torch.float32, device="cuda")    # the guard is only raised
    FU.attn_pad_correct(o, lse, npad, rows, big, out)
    assert float(big) == 1e3
    buf = torch.full((B, rows, H * 128 + 48), 7.0, dtype=torch.bfloat16, device="cuda")
    FU.attn_pad_correct(o, lse, npad, rows, guard, buf[:, :, 16:16 + H * 128])
    torch.cuda.synchronize()
    assert torch.equal(buf[:, :, 16:16 + H * 128], ref)
    assert bool((buf[:, :, :16] == 7.0).all()) and bool((buf[:, :, 16 + H * 128:] == 7.0).all())


def test_attn_pad_correct_errors_are_reported():
    o = torch.zeros((1, 2, 8, 128), dtype=torch.bfloat16, device="cuda")
    lse = torch.zeros((1, 2, 8), device="cuda")
    npad = torch.ones(1, device="cuda")
    guard = torch.zeros((), device="cuda")
    out = torch.empty((1, 4, 256), dtype=torch.bfloat16, device="cuda")
    lib = mold_amd.load()
    rc = lib.mq_attn_pad_correct(o.data_ptr(), 1, 2, 4, o.stride(0), o.stride(1), o.stride(2), lse.data_ptr(),
                                 lse.stride(0), lse.stride(1), npad.data_ptr(), out.data_ptr(), out.stride(0), 200,
                                 guard.data_ptr(), None)
    assert rc == -1 and b"ldo" in lib.mq_last_error()
    rc = lib.mq_attn_pad_correct(o.data_ptr(), 1, 2, 4, o.stride(0), o.stride(1), 132, lse.data_ptr(),
                                 lse.stride(0), lse.stride(1), npad.data_ptr(), out.data_ptr(), out.stride(0), 256,
                                 guard.data_ptr(), None)
    assert rc == -1 and b"multiples of 8" in lib.mq_last_error()
    with pytest.raises(ValueError):   # more rows than o holds
        FU.attn_pad_correct(o, lse, npad, 9, guard, torch.empty((1, 9, 256), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):   # lse of the wrong head count
        FU.attn_pad_correct(o, lse[:, :1], npad, 4, guard, out)


def test_glue_errors_are_reported():
    mold_amd.load()
    y = torch.zeros((4, 3 * 128), device="cuda")
    cs = torch.zeros((4, 64), device="cuda")
    w = torch.ones(128, dtype=torch.bfloat16, device="cuda")
    q, k, v = FU.new_heads(1, 4, "cuda")
    lib = mold_amd.load()
    rc = lib.mq_qk_norm_rope(y.data_ptr(), 0, y.stride(0), 4, 1, 64, w.data_ptr(), w.data_ptr(), 1e-6,
                             cs.data_ptr(), cs.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), 0, 4, None)
    assert rc == -1 and b"head_dim" in lib.mq_last_error()
    with pytest.raises(MoldqError):   # row range past the joint sequence
        FU.qk_norm_rope(y, 1, w, w, cs, cs, q, k, v, 2)
    x = torch.zeros((2, 6), device="cuda")
    with pytest.raises(ValueError):
        FU.adaln_modulate(x, torch.zeros(5, device="cuda"), torch.zeros(5, device="cuda"))
    with pytest.raises(MoldqError):   # cols not a multiple of 4
        FU.adaln_modulate(x, torch.zeros(6, device="cuda"), torch.zeros(6, device="cuda"))
