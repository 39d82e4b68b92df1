"""Gated attention with pair bias on the GPU against the oracle
(oracle/ref.py attention, AttentionGpu.run restated in float64).

The four cases of test/evoformer-attention.gpu.test.ts:33-50: MSA row
attention with a separate pair bias, MSA column attention (transposed, no
bias), triangle attention starting node (normalized-input bias) and ending
node (transposed, normalized-input bias). That test's block-0 fixture is not
in the reference tree, so the inputs are seeded synthetic tensors of the
same roles; its bar (mean absolute error < 2e-5, max < 3e-4) holds for the
f32 path, together with 1e-5 of the largest output. The f16 path (the MFMA
flash kernel at head dimension 32, AlphaFold's widths) is held to 1e-2 of
the largest output.
"""
import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch

    from afhip import device

    device.open_device(0)
    return torch.device("cuda", 0)


def weights(seed, C, H, pair=None, Cp=0):
    w = {"queryNormScale": ref.normal(seed, (C,), 0.01, 1.0), "queryNormOffset": ref.normal(seed + 1, (C,), 0.01),
         "queryWeight": ref.normal(seed + 2, (C, C), 1 / C), "keyWeight": ref.normal(seed + 3, (C, C), 1 / C),
         "valueWeight": ref.normal(seed + 4, (C, C), 1 / C), "gatingWeight": ref.normal(seed + 5, (C, C), 1 / C),
         "gatingBias": ref.normal(seed + 6, (C,), 0.1, 1.0), "outputWeight": ref.normal(seed + 7, (C, C), 1 / C),
         "outputBias": ref.normal(seed + 8, (C,), 0.01)}
    pb = None
    if pair == "separate":
        pb = {"source": "separate", "channels": Cp, "layerNormScale": ref.normal(seed + 9, (Cp,), 0.01, 1.0),
              "layerNormOffset": ref.normal(seed + 10, (Cp,), 0.01),
              "projectionWeight": ref.normal(seed + 11, (Cp, H), 1 / Cp)}
    elif pair == "normalized-input":
        pb = {"source": "normalized-input", "projectionWeight": ref.normal(seed + 11, (C, H), 1 / C)}
    return w, pb


def case(name, S, L, C, H, Cp=0, seed=0xA7700):
    """Inputs of one reference case: (activations, mask, batch, queries,
    transpose, weights, pair_bias). MSA cases take activations [S][L][C]
    and the MSA mask; triangle cases [L][L][C] and the pair mask."""
    msa = name.startswith("msa")
    rows = (S if msa else L) * L
    x = ref.normal(seed, (rows, C))
    mask = (ref.uniform(seed + 1, (rows,), 0, 1) > 0.2).astype(np.float32)
    mask[:L] = 0.0  # one fully masked stretch: a row of keys entirely masked
    pair = {"msa_row": "separate", "msa_column": None, "triangle_start": "normalized-input",
            "triangle_end": "normalized-input"}[name]
    w, pb = weights(seed + 10, C, H, pair, Cp)
    if pair == "separate":
        pb["activations"] = ref.normal(seed + 2, (L * L * Cp,))
    transpose = name in ("msa_column", "triangle_end")
    first = S if msa else L
    batch, queries = (L, first) if transpose else (first, L)
    return x, mask, batch, queries, transpose, w, pb


CASES = ["msa_row", "msa_column", "triangle_start", "triangle_end"]


def run_case(dev, x, mask, B, Q, C, H, transpose, w, pb, precision="f32", in_dtype="f32", out_dtype="f32",
             residual=None):
    import torch

    from afhip import attention

    op = attention.Attention(B, Q, C, H, transpose=transpose, pair_bias=None if pb is None else pb["source"],
                             pair_channels=pb["channels"] if pb is not None and pb["source"] == "separate" else 0,
                             precision=precision, in_dtype=in_dtype, out_dtype=out_dtype,
                             residual=residual is not None)
    op.prepare(attention.pack_weights(w, pb))
    tdt = torch.float16 if in_dtype == "f16" else torch.float32
    xt = torch.from_numpy(x.reshape(B * Q, C)).to(dev, tdt)
    mt = torch.from_numpy(mask).to(dev)
    pt = None
    if pb is not None and pb["source"] == "separate":
        pt = torch.from_numpy(np.asarray(pb["activations"], np.float32)).to(dev, tdt)
    out = None
    if residual is not None:
        out = torch.from_numpy(residual.reshape(B * Q, C)).to(dev, torch.float16 if out_dtype == "f16" else torch.float32)
    out = op(xt, mt, pt, out=out)
    torch.cuda.synchronize()
    return out.float().cpu().numpy().reshape(-1)


@pytest.mark.parametrize("name", CASES)
def test_reference_cases_f32(dev, name):
    # head dimension 8 (the general kernel), ragged lengths
    x, mask, B, Q, tr, w, pb = case(name, S=5, L=19, C=32, H=4, Cp=12)
    expect = ref.attention(x, mask, w, B, Q, 32, 4, transpose=tr, pair_bias=pb)
    got = run_case(dev, x, mask, B, Q, 32, 4, tr, w, pb)
    m = ref.error_metrics(got, expect)
    assert m["meanAbsoluteError"] < 2e-5 and m["maxAbsoluteError"] < 3e-4
    assert m["maxAbsoluteError"] <= 1e-5 * np.abs(expect).max()


def test_attention_gpu_run_mirrors_the_reference_call(dev):
    # AttentionGpu.run over host arrays, as the reference's test calls it.
    from afhip import attention

    x, mask, B, Q, tr, w, pb = case("msa_row", S=3, L=11, C=16, H=2, Cp=8)
    inp = {"activations": x.reshape(-1), "mask": mask, "batch": B, "queryLength": Q, "channels": 16, "heads": 2,
           "transpose": tr, "weights": w, "pairBias": pb}
    res = attention.AttentionGpu().run(inp)
    expect = ref.attention(x, mask, w, B, Q, 16, 2, transpose=tr, pair_bias=pb)
    assert np.abs(res["output"] - expect).max() <= 1e-5 * np.abs(expect).max()
    assert res["elapsedMilliseconds"] >= 0 and res["memory"]["currentBytes"] > 0
    bad = dict(inp, heads=3)
    with pytest.raises(attention._lib.RangeError, match="integral head dimension"):
        attention.AttentionGpu().run(bad)
    with pytest.raises(attention._lib.RangeError, match="mask has 32 values; expected 33"):
        attention.AttentionGpu().run(dict(inp, mask=mask[:-1]))


@pytest.mark.parametrize("C,H", [(32, 1), (15, 3), (64, 2), (24, 24)])
def test_general_head_dimensions_f32(dev, C, H):
    # head dimensions 32, 5, 32 and 1 through the general kernel's instances
    x, mask, B, Q, tr, w, pb = case("triangle_start", S=0, L=13, C=C, H=H)
    expect = ref.attention(x, mask, w, B, Q, C, H, transpose=tr, pair_bias=pb)
    got = run_case(dev, x, mask, B, Q, C, H, tr, w, pb)
    assert np.abs(got - expect).max() <= 1e-5 * np.abs(expect).max()


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("in_dtype", ["f32", "f16"])
def test_reference_cases_f16_mfma(dev, name, in_dtype):
    # AlphaFold's widths: MSA attention c_m 256 over 8 heads, triangle
    # attention c_z 128 over 4 heads, head dimension 32 (the MFMA flash
    # kernel); 70 residues, so both the query and the key tiles are ragged.
    msa = name.startswith("msa")
    C, H = (256, 8) if msa else (128, 4)
    x, mask, B, Q, tr, w, pb = case(name, S=9, L=70, C=C, H=H, Cp=128, seed=0xA7800)
    if in_dtype == "f16":
        x = ref.round_f16(x)
        if pb is not None and pb["source"] == "separate":
            pb["activations"] = ref.round_f16(pb["activations"])
    expect = ref.attention(x, mask, w, B, Q, C, H, transpose=tr, pair_bias=pb)
    got = run_case(dev, x, mask, B, Q, C, H, tr, w, pb, precision="f16", in_dtype=in_dtype, out_dtype="f16")
    assert np.abs(got - expect).max() <= 1e-2 * np.abs(expect).max()


def test_f16_long_keys_and_residual(dev):
    # 300 keys (ten key blocks, the last ragged; three query blocks of 128),
    # transposed with two batch entries, the second entirely masked, and the
    # result added onto the output in place.
    C, H, B, Q = 128, 4, 2, 300
    w, _ = weights(0xA7900, C, H)
    x = ref.normal(0xA7901, (Q * B, C))
    mask = (ref.uniform(0xA7902, (Q, B), 0, 1) > 0.3).astype(np.float32)
    mask[:, 1] = 0.0
    mask = mask.reshape(-1)
    base = ref.round_f16(ref.normal(0xA7903, (Q * B, C)))
    expect = base.reshape(-1) + ref.attention(x, mask, w, B, Q, C, H, transpose=True)
    got = run_case(dev, x, mask, B, Q, C, H, True, w, None, precision="f16", out_dtype="f16", residual=base)
    assert np.abs(got - expect).max() <= 1e-2 * np.abs(expect).max()


@pytest.mark.parametrize("name", ["triangle_start", "msa_column", "msa_row"])
def test_f16_sharp_logits_move_the_offset(dev, name):
    # Logits spread over tens of units, so a row's running offset moves in
    # middle key blocks and the fast probability check fails there (the exact
    # step redoes the block). The spread comes from the pair bias scaled by
    # 20 (f32 all the way, so the f16 operands add no error beyond the usual),
    # and for column attention, which has no pair bias, from the queries
    # scaled by 4. 200 keys (150 for MSA row attention): seven key blocks, the
    # last ragged, with masked keys and a fully masked stretch.
    msa = name.startswith("msa")
    C, H = (256, 8) if msa else (128, 4)
    x, mask, B, Q, tr, w, pb = case(name, S=200 if msa else 0, L=150 if msa else 200, C=C, H=H, Cp=64,
                                    seed=0xA7E00)
    if pb is not None:
        pb["projectionWeight"] = pb["projectionWeight"] * 20.0
    else:
        w["queryWeight"] = w["queryWeight"] * 4.0
    x = ref.round_f16(x)
    if pb is not None and pb["source"] == "separate":
        pb["activations"] = ref.round_f16(pb["activations"])
    expect = ref.attention(x, mask, w, B, Q, C, H, transpose=tr, pair_bias=pb)
    got = run_case(dev, x, mask, B, Q, C, H, tr, w, pb, precision="f16", in_dtype="f16", out_dtype="f16")
    assert np.abs(got - expect).max() <= 1e-2 * np.abs(expect).max()


def test_single_query_and_fully_masked(dev):
    # One query: softmax over one key; a fully masked batch entry averages
    # its values (every logit clamps to -1e8).
    C, H = 64, 2
    w, _ = weights(0xA7A00, C, H)
    for prec in ("f32", "f16"):
        x = ref.normal(0xA7A10, (3, C))
        mask = np.array([1, 0, 1], np.float32)
        expect = ref.attention(x, mask, w, 3, 1, C, H)
        got = run_case(dev, x, mask, 3, 1, C, H, False, w, None, precision=prec)
        assert np.abs(got - expect).max() <= (1e-2 if prec == "f16" else 1e-5) * np.abs(expect).max()
        x = ref.normal(0xA7A20, (40, C))
        mask = np.zeros(40, np.float32)
        expect = ref.attention(x, mask, w, 1, 40, C, H)
        got = run_case(dev, x, mask, 1, 40, C, H, False, w, None, precision=prec)
        assert np.abs(got - expect).max() <= (1e-2 if prec == "f16" else 1e-5) * np.abs(expect).max()


def test_workspace_and_operands_are_checked(dev):
    import ctypes

    import torch

    from afhip import _lib, attention
    from afhip.device import ptr, stream_handle

    op = attention.Attention(4, 4, 16, 2, pair_bias="separate", pair_channels=8)
    x = torch.zeros((16, 16), device=dev)
    m = torch.ones(16, device=dev)
    with pytest.raises(_lib.RangeError, match="needs its pair activations"):
        op(x, m, None)
    out = torch.empty_like(x)
    with pytest.raises(_lib.RangeError, match="workspace of 16 bytes"):
        _lib.call("afhip_attention_run", ctypes.byref(op.desc), ptr(x), ptr(m), ptr(x), ptr(op.prepared), ptr(out),
                  ptr(op.workspace), 16, stream_handle())


def test_full_size_ending_node_is_transposed_starting_node(dev):
    # At the headline's size (L = 384, c_z 128, 4 heads, f16): triangle
    # attention around the ending node of z equals the starting node applied
    # to z transposed, transposed back, bit for bit -- the same rows reach the
    # same kernels in the same attention order.
    import torch

    from afhip import attention

    L, C, H = 384, 128, 4
    w, pb = weights(0xA7B00, C, H, "normalized-input")
    z = torch.from_numpy(ref.round_f16(ref.normal(0xA7B10, (L, L, C)))).half().to(dev)
    mask = torch.from_numpy((ref.uniform(0xA7B11, (L, L), 0, 1) > 0.1).astype(np.float32)).to(dev)
    packed = attention.pack_weights(w, pb)
    outs = []
    for tp, zz, mm in ((True, z, mask), (False, z.transpose(0, 1).contiguous(), mask.t().contiguous())):
        op = attention.Attention(L, L, C, H, transpose=tp, pair_bias="normalized-input", precision="f16",
                                 in_dtype="f16", out_dtype="f16")
        op.prepare(packed)
        outs.append(op(zz.reshape(L * L, C), mm.reshape(-1)).reshape(L, L, C))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1].transpose(0, 1))
    assert torch.isfinite(outs[0].float()).all()


def test_full_size_msa_row_attention_commutes_with_sequence_order(dev):
    # MSA row attention at N_seq 512 x N_res 256 (c_m 256, 8 heads, pair bias
    # from a [256, 256, 128] pair): permuting the sequences permutes the
    # output, bit for bit, although a workgroup pairs two sequences.
    import torch

    from afhip import attention

    S, L, C, H, Cp = 512, 256, 256, 8, 128
    w, pb = weights(0xA7C00, C, H, "separate", Cp)
    x = torch.from_numpy(ref.round_f16(ref.normal(0xA7C10, (S, L, C)))).half().to(dev)
    mask = torch.from_numpy((ref.uniform(0xA7C11, (S, L), 0, 1) > 0.1).astype(np.float32)).to(dev)
    pair = torch.from_numpy(ref.round_f16(ref.normal(0xA7C12, (L * L * Cp,)))).half().to(dev)
    perm = torch.from_numpy(np.random.default_rng(5).permutation(S)).to(dev)
    op = attention.Attention(S, L, C, H, pair_bias="separate", pair_channels=Cp, precision="f16", in_dtype="f16",
                             out_dtype="f16")
    op.prepare(attention.pack_weights(w, pb))
    a = op(x.reshape(S * L, C), mask.reshape(-1), pair).reshape(S, L, C).clone()
    b = op(x[perm].contiguous().reshape(S * L, C), mask[perm].contiguous().reshape(-1), pair).reshape(S, L, C)
    torch.cuda.synchronize()
    assert torch.equal(a[perm], b)
    assert torch.isfinite(a.float()).all()


@pytest.mark.parametrize("name,S,L,C,H", [("msa_row", 11, 70, 192, 6), ("msa_column", 11, 37, 192, 6),
                                          ("msa_row", 13, 45, 256, 8), ("msa_column", 12, 37, 256, 8)])
def test_f16_head_groups_and_odd_batches(dev, name, S, L, C, H):
    # The head-dimension-32 kernel orders its workgroups in groups of four
    # heads when the head count allows (8 here) and batch pair by batch pair
    # otherwise (6); an odd number of batch entries leaves the last
    # workgroup's second entry empty, whose mask-code row lies past the
    # codes (column attention: 37 batch entries).
    x, mask, B, Q, tr, w, pb = case(name, S=S, L=L, C=C, H=H, Cp=32, seed=0xA8100)
    x = ref.round_f16(x)
    if pb is not None and pb["source"] == "separate":
        pb["activations"] = ref.round_f16(pb["activations"])
    expect = ref.attention(x, mask, w, B, Q, C, H, transpose=tr, pair_bias=pb)
    got = run_case(dev, x, mask, B, Q, C, H, tr, w, pb, precision="f16", in_dtype="f16", out_dtype="f16")
    assert np.abs(got - expect).max() <= 1e-2 * np.abs(expect).max()


@pytest.mark.parametrize("name,B,Q,C,H,Cp", [("triangle_start", 384, 384, 128, 4, 0), ("msa_row", 512, 256, 256, 8, 128),
                                              ("triangle_start", 77, 77, 128, 4, 0)])
def test_f16_residual_adds_the_rounded_output(dev, name, B, Q, C, H, Cp):
    # With the residual, out = f16(old + f16(attention)), f32 sum: at c = 128
    # the output projection's streaming kernel adds into the output itself
    # (reading the old values a tile ahead of its stores; full size gives
    # each workgroup nine passes, 77 x 77 a ragged last tile), at c = 256 a
    # second pass does. Either way bit for bit the two steps done apart.
    import torch

    from afhip import attention

    pair = "normalized-input" if name.startswith("triangle") else "separate"
    w, pb = weights(0xA7F00, C, H, pair, Cp)
    x = torch.from_numpy(ref.round_f16(ref.normal(0xA7F10, (B * Q, C)))).half().to(dev)
    mask = torch.from_numpy((ref.uniform(0xA7F11, (B * Q,), 0, 1) > 0.1).astype(np.float32)).to(dev)
    p = None
    if pair == "separate":
        p = torch.from_numpy(ref.round_f16(ref.normal(0xA7F12, (Q * Q * Cp,)))).half().to(dev)
    packed = attention.pack_weights(w, pb)
    kw = dict(pair_bias=pair, pair_channels=Cp, precision="f16", in_dtype="f16", out_dtype="f16")
    plain = attention.Attention(B, Q, C, H, **kw)
    plain.prepare(packed)
    y = plain(x, mask, p).clone()
    old = torch.from_numpy(ref.round_f16(ref.normal(0xA7F13, (B * Q, C)))).half().to(dev)
    res = attention.Attention(B, Q, C, H, residual=True, **kw)
    res.prepare(packed)
    out = old.clone()
    res(x, mask, p, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, (old.float() + y.float()).half())


@pytest.mark.parametrize("name", ["msa_row", "msa_column", "triangle_start", "triangle_end"])
@pytest.mark.parametrize("C,H", [(64, 8), (64, 4), (96, 4)])
def test_f16_mfma_narrow_heads(dev, name, C, H):
    # Head dimensions 8, 16 and 24 on the f16 MFMA kernel (each head padded to
    # 32 channels with zeros): extra-MSA row attention is c_e 64 over 8 heads.
    x, mask, B, Q, tr, w, pb = case(name, S=7, L=45, C=C, H=H, Cp=64, seed=0xA7D00)
    expect = ref.attention(x, mask, w, B, Q, C, H, transpose=tr, pair_bias=pb)
    got = run_case(dev, x, mask, B, Q, C, H, tr, w, pb, precision="f16", out_dtype="f16")
    assert np.abs(got - expect).max() <= 1e-2 * np.abs(expect).max()
