"""The execution layer on the GPU: the pooled allocator over device memory
(src/runtime/allocator.ts:168-388; the policy itself is checked on the CPU by
test_execution_pool.py), addInPlace (src/runtime/execution.ts:415-450), and
the pair steps of an Evoformer block chained on the device
(src/evoformer/block.ts:1683-1750) against the same operators called one by
one and against the oracle composed the same way."""
import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.gpu

MiB = 1 << 20


@pytest.fixture(scope="module")
def dev():
    import torch

    from afhip import device

    device.open_device(0)
    return torch.device("cuda", 0)


def test_allocator_reuses_budgets_and_frees(dev):
    from afhip import _lib
    from afhip.execution import Execution, memory_resident, set_memory_budget

    base = memory_resident()
    ex = Execution()
    p = ex.allocate("scratch-1", 3 * MiB)
    ex.release_tensor(p)
    assert ex.allocate("scratch-2", 5 * MiB // 2) == p  # 2.5 MiB takes the idle 3 MiB
    snap = ex.snapshot()
    assert snap["residentBytes"] == 3 * MiB and snap["bufferCount"] == 1 and snap["allocationCount"] == 2
    assert snap["peakComposition"][0]["label"] == "scratch"
    q = ex.allocate("small", 1000)  # the pool holds nothing for it
    assert q != p and ex.snapshot()["residentBytes"] == 3 * MiB + 1000
    assert memory_resident() == base + 3 * MiB + 1000
    # the budget counts every execution's resident bytes and names the tensor
    set_memory_budget(memory_resident() + MiB)
    try:
        with pytest.raises(_lib.AfhipError, match="GPU memory budget exceeded.*for pair-update"):
            ex.allocate("pair-update", 4 * MiB)
    finally:
        set_memory_budget(None)
    # checkpoints, then idle buffers leave after four submitted boundaries
    mark = ex.checkpoint()
    ex.allocate("window-0", 2 * MiB)
    ex.allocate("window-1", 2 * MiB)
    ex.release_since(mark)
    assert ex.snapshot()["pooledBytes"] == 4 * MiB
    for _ in range(4):
        ex.note_submitted()
    snap = ex.snapshot()
    assert snap["pooledBytes"] == 0 and snap["residentBytes"] == 3 * MiB + 1000
    with pytest.raises(_lib.RangeError, match="not a live tensor"):
        ex.release_tensor(12345)
    ex.release()
    assert memory_resident() == base


def test_upload_and_add_in_place(dev):
    from afhip.execution import Execution

    ex = Execution()
    n = 100003
    a = ref.normal(1, (n,))
    b = ref.round_f16(ref.normal(2, (n,)))
    pa = ex.upload("base", a)
    pb = ex.upload("update", b.astype(np.float16))
    ex.add_in_place(pa, pb, n, "f32", "f16")
    got = ex.download(pa, (n,))
    assert np.array_equal(got, (a + b).astype(np.float32))
    h = ex.upload("half", ref.round_f16(a).astype(np.float16))
    ex.add_in_place(h, pb, n, "f16", "f16")
    expect = ref.round_f16(ref.round_f16(a) + b)
    assert np.array_equal(ex.download(h, (n,), np.float16).astype(np.float32), expect)
    ex.release()


def _block_weights(seed, cz, ch, cm, co, h):
    from bench import triangle_weights

    opm_w = {"layerNormScale": ref.normal(seed, (cm,), 0.01, 1.0), "layerNormOffset": ref.normal(seed + 1, (cm,), 0.01),
             "leftWeight": ref.normal(seed + 2, (cm, co), 1 / cm), "leftBias": ref.normal(seed + 3, (co,), 0.02),
             "rightWeight": ref.normal(seed + 4, (cm, co), 1 / cm), "rightBias": ref.normal(seed + 5, (co,), 0.02),
             "outputWeight": ref.normal(seed + 6, (co * co, cz), 1 / (co * co)),
             "outputBias": ref.normal(seed + 7, (cz,), 0.02)}
    tr_w = {"layerNormScale": ref.normal(seed + 8, (cz,), 0.01, 1.0), "layerNormOffset": ref.normal(seed + 9, (cz,), 0.01),
            "firstWeight": ref.normal(seed + 10, (cz, h), 1 / cz), "firstBias": ref.normal(seed + 11, (h,), 0.02),
            "secondWeight": ref.normal(seed + 12, (h, cz), 1 / h), "secondBias": ref.normal(seed + 13, (cz,), 0.02)}
    def att(s0):
        a = {"queryNormScale": ref.normal(s0, (cz,), 0.01, 1.0), "queryNormOffset": ref.normal(s0 + 1, (cz,), 0.01),
             "queryWeight": ref.normal(s0 + 2, (cz, cz), 1 / cz), "keyWeight": ref.normal(s0 + 3, (cz, cz), 1 / cz),
             "valueWeight": ref.normal(s0 + 4, (cz, cz), 1 / cz), "gatingWeight": ref.normal(s0 + 5, (cz, cz), 1 / cz),
             "gatingBias": ref.normal(s0 + 6, (cz,), 0.1, 1.0), "outputWeight": ref.normal(s0 + 7, (cz, cz), 1 / cz),
             "outputBias": ref.normal(s0 + 8, (cz,), 0.01)}
        return {"heads": 4, "attention": a, "pairProjectionWeight": ref.normal(s0 + 9, (cz, 4), 1 / cz)}

    return {"outerProductMean": opm_w, "triangleMultiplicationOutgoing": triangle_weights(seed + 20, cz, ch),
            "triangleMultiplicationIncoming": triangle_weights(seed + 40, cz, ch),
            "triangleAttentionStarting": att(seed + 60), "triangleAttentionEnding": att(seed + 80),
            "pairTransition": tr_w}


def test_pair_stack_is_the_operators_in_sequence(dev):
    # f16 at AlphaFold's widths (the fused kernels): the chained stack gives
    # the result of the six operators called one after another on the same
    # pair, bit for bit, with its workspaces drawn from the pool.
    import torch

    from afhip import attention, opm, transition, triangle
    from afhip.execution import Execution, PairStack

    L, S, cm, co, cz, ch = 64, 16, 64, 32, 128, 128
    w = _block_weights(0xAF2100, cz, ch, cm, co, 4 * cz)
    msa = torch.from_numpy(ref.round_f16(ref.normal(1, (S, L, cm)))).half().to(dev)
    msa_mask = torch.from_numpy((ref.uniform(2, (S, L), 0, 1) > 0.1).astype(np.float32)).to(dev)
    pair_mask = torch.from_numpy((ref.uniform(3, (L, L), 0, 1) > 0.15).astype(np.float32)).to(dev)
    pair0 = torch.from_numpy(ref.round_f16(ref.normal(4, (L, L, cz)))).half().to(dev)

    expect = pair0.clone()
    o = opm.OuterProductMean(S, L, cm, co, cz, precision="f16", msa_dtype="f16", out_dtype="f16", residual=True)
    o.prepare(w["outerProductMean"])
    o(msa, msa_mask, out=expect)
    for d, key in (("outgoing", "triangleMultiplicationOutgoing"), ("incoming", "triangleMultiplicationIncoming")):
        t = triangle.TriangleMultiplication(L, cz, ch, direction=d, precision="f16", pair_dtype="f16",
                                            out_dtype="f16", residual=True)
        t.prepare(w[key])
        t(expect, pair_mask, out=expect)
    for tp, key in ((False, "triangleAttentionStarting"), (True, "triangleAttentionEnding")):
        a = attention.Attention(L, L, cz, 4, transpose=tp, pair_bias="normalized-input", precision="f16",
                                in_dtype="f16", out_dtype="f16", residual=True)
        a.prepare(attention.pack_weights(w[key]["attention"], {"source": "normalized-input",
                                                              "projectionWeight": w[key]["pairProjectionWeight"]}))
        flat = expect.reshape(L * L, cz)
        a(flat, pair_mask.reshape(-1), out=flat)
    tr = transition.Transition(L * L, cz, 4 * cz, precision="f16", in_dtype="f16", out_dtype="f16", residual=True)
    tr.prepare(w["pairTransition"])
    tr(expect, out=expect)

    ex = Execution()
    stack = PairStack(ex, L, sequences=S, c_m=cm, c_z=cz, c_outer=co, c_hidden=ch)
    stack.prepare(w)
    pair = pair0.clone()
    stack(pair, pair_mask, msa, msa_mask)
    torch.cuda.synchronize()
    assert torch.equal(pair, expect)
    snap = ex.snapshot()
    # Only the prepared weights stay live; the steps' workspaces went back to
    # the pool, and the peak held the weights and one step's workspace.
    weights = sum(e["bytes"] for e in snap["peakComposition"] if e["label"].endswith(".weights"))
    assert snap["currentBytes"] == weights > 0
    assert sum(1 for e in snap["peakComposition"] if not e["label"].endswith(".weights")) == 1
    ex.release()


def test_pair_stack_against_the_oracle(dev):
    # f32 at small widths (the general kernels) against the oracle composed in
    # the block's order: z += OPM(m); z += outgoing(z); z += incoming(z);
    # z += attention_start(z); z += attention_end(z); z += transition(z).
    from afhip.execution import Execution, PairStack

    L, S, cm, co, cz, ch = 24, 8, 16, 8, 32, 32
    w = _block_weights(0xAF2200, cz, ch, cm, co, 4 * cz)
    msa = ref.normal(5, (S, L, cm))
    msa_mask = (ref.uniform(6, (S, L), 0, 1) > 0.1).astype(np.float32)
    pair_mask = (ref.uniform(7, (L, L), 0, 1) > 0.15).astype(np.float32)
    z = ref.normal(8, (L, L, cz))
    expect = z + ref.opm(msa, msa_mask, w["outerProductMean"])
    expect = expect + ref.triangle("outgoing", expect, pair_mask, w["triangleMultiplicationOutgoing"])
    expect = expect + ref.triangle("incoming", expect, pair_mask, w["triangleMultiplicationIncoming"])
    for tp, key in ((False, "triangleAttentionStarting"), (True, "triangleAttentionEnding")):
        pb = {"source": "normalized-input", "projectionWeight": w[key]["pairProjectionWeight"]}
        expect = expect + ref.attention(expect, pair_mask, w[key]["attention"], L, L, cz, 4, transpose=tp,
                                        pair_bias=pb).reshape(L, L, cz)
    expect = expect + ref.transition(expect.reshape(L * L, cz), w["pairTransition"]).reshape(L, L, cz)

    ex = Execution()
    stack = PairStack(ex, L, sequences=S, c_m=cm, c_z=cz, c_outer=co, c_hidden=ch, precision="f32",
                      pair_dtype="f32", msa_dtype="f32")
    stack.prepare(w)
    pm, pmm = ex.upload("msa", msa), ex.upload("msa-mask", msa_mask)
    pz, pzm = ex.upload("pair", z), ex.upload("pair-mask", pair_mask)
    stack(pz, pzm, pm, pmm)
    got = ex.download(pz, (L, L, cz))
    assert np.abs(got - expect).max() <= 1e-4 * np.abs(expect).max()
    ex.release()


def test_pair_stack_rejects_mismatched_attention(dev):
    from afhip import _lib
    from afhip.execution import Execution, PairStack

    ex = Execution()
    stack = PairStack(ex, 16, sequences=4, c_m=16, c_z=32, c_outer=8, c_hidden=32, precision="f32",
                      pair_dtype="f32", msa_dtype="f32")
    stack.desc.attention_end.channels = 64
    stack.weights.attention_end = 1  # never read: the shapes are checked first
    pz = ex.allocate("pair", 16 * 16 * 32 * 4)
    pm = ex.allocate("pair-mask", 16 * 16 * 4)
    with pytest.raises(_lib.RangeError, match="triangle attention does not match"):
        stack(pz, pm)
    ex.release()


def test_pair_stack_rejects_mismatched_steps(dev):
    from afhip import _lib
    from afhip.execution import Execution, PairStack

    ex = Execution()
    stack = PairStack(ex, 16, sequences=4, c_m=16, c_z=32, c_outer=8, c_hidden=32, precision="f32",
                      pair_dtype="f32", msa_dtype="f32")
    stack.desc.transition.channels = 16
    stack.weights.transition = 1  # never read: the shapes are checked first
    pz = ex.allocate("pair", 16 * 16 * 32 * 4)
    pm = ex.allocate("pair-mask", 16 * 16 * 4)
    with pytest.raises(_lib.RangeError, match="transition does not match"):
        stack(pz, pm)
    ex.release()


def _msa_weights(seed, cm, cz, heads=8):
    def att(s0):
        return {"queryNormScale": ref.normal(s0, (cm,), 0.01, 1.0), "queryNormOffset": ref.normal(s0 + 1, (cm,), 0.01),
                "queryWeight": ref.normal(s0 + 2, (cm, cm), 1 / cm), "keyWeight": ref.normal(s0 + 3, (cm, cm), 1 / cm),
                "valueWeight": ref.normal(s0 + 4, (cm, cm), 1 / cm),
                "gatingWeight": ref.normal(s0 + 5, (cm, cm), 1 / cm), "gatingBias": ref.normal(s0 + 6, (cm,), 0.1, 1.0),
                "outputWeight": ref.normal(s0 + 7, (cm, cm), 1 / cm), "outputBias": ref.normal(s0 + 8, (cm,), 0.01)}
    return {"msaRowAttention": {"attention": att(seed), "pairLayerNormScale": ref.normal(seed + 20, (cz,), 0.01, 1.0),
                                "pairLayerNormOffset": ref.normal(seed + 21, (cz,), 0.01),
                                "pairProjectionWeight": ref.normal(seed + 22, (cz, heads), 1 / cz)},
            "msaColumnAttention": {"attention": att(seed + 40)},
            "msaTransition": {"layerNormScale": ref.normal(seed + 60, (cm,), 0.01, 1.0),
                              "layerNormOffset": ref.normal(seed + 61, (cm,), 0.01),
                              "firstWeight": ref.normal(seed + 62, (cm, 4 * cm), 1 / cm),
                              "firstBias": ref.normal(seed + 63, (4 * cm,), 0.02),
                              "secondWeight": ref.normal(seed + 64, (4 * cm, cm), 1 / (4 * cm)),
                              "secondBias": ref.normal(seed + 65, (cm,), 0.02)}}


def _oracle_block(msa, msa_mask, z, pair_mask, w, S, L, cm, cz, opm_first, heads=8):
    m, z = msa.astype(np.float64), z.astype(np.float64)
    if opm_first:
        z = z + ref.opm(m, msa_mask, w["outerProductMean"])
    row = w["msaRowAttention"]
    pb = {"source": "separate", "activations": z, "channels": cz, "layerNormScale": row["pairLayerNormScale"],
          "layerNormOffset": row["pairLayerNormOffset"], "projectionWeight": row["pairProjectionWeight"]}
    m = m + ref.attention(m, msa_mask, row["attention"], S, L, cm, heads, pair_bias=pb).reshape(S, L, cm)
    m = m + ref.attention(m, msa_mask, w["msaColumnAttention"]["attention"], L, S, cm, heads,
                          transpose=True).reshape(S, L, cm)
    m = m + ref.transition(m.reshape(S * L, cm), w["msaTransition"]).reshape(S, L, cm)
    if not opm_first:
        z = z + ref.opm(m, msa_mask, w["outerProductMean"])
    z = z + ref.triangle("outgoing", z, pair_mask, w["triangleMultiplicationOutgoing"])
    z = z + ref.triangle("incoming", z, pair_mask, w["triangleMultiplicationIncoming"])
    for tp, key in ((False, "triangleAttentionStarting"), (True, "triangleAttentionEnding")):
        pbz = {"source": "normalized-input", "projectionWeight": w[key]["pairProjectionWeight"]}
        z = z + ref.attention(z, pair_mask, w[key]["attention"], L, L, cz, 4, transpose=tp,
                              pair_bias=pbz).reshape(L, L, cz)
    z = z + ref.transition(z.reshape(L * L, cz), w["pairTransition"]).reshape(L, L, cz)
    return m, z


@pytest.mark.parametrize("opm_first", [False, True])
def test_evoformer_block_against_the_oracle(dev, opm_first):
    # f32 at small widths: the whole block against the oracle composed in the
    # block's order (block.ts:1673-1759).
    from afhip.execution import EvoformerBlock, Execution

    L, S, cm, co, cz, ch = 20, 6, 32, 8, 32, 32
    w = _block_weights(0xAF2300, cz, ch, cm, co, 4 * cz)
    w.update(_msa_weights(0xAF2400, cm, cz))
    msa = ref.normal(9, (S, L, cm))
    msa_mask = (ref.uniform(10, (S, L), 0, 1) > 0.1).astype(np.float32)
    pair_mask = (ref.uniform(11, (L, L), 0, 1) > 0.15).astype(np.float32)
    z = ref.normal(12, (L, L, cz))
    em, ez = _oracle_block(msa, msa_mask, z, pair_mask, w, S, L, cm, cz, opm_first)
    ex = Execution()
    blk = EvoformerBlock(ex, L, sequences=S, c_m=cm, c_z=cz, c_outer=co, c_hidden=ch, opm_first=opm_first,
                         precision="f32", dtype="f32")
    blk.prepare(w)
    pm, pmm = ex.upload("msa", msa), ex.upload("msa-mask", msa_mask)
    pz, pzm = ex.upload("pair", z), ex.upload("pair-mask", pair_mask)
    blk(pm, pmm, pz, pzm)
    gm, gz = ex.download(pm, (S, L, cm)), ex.download(pz, (L, L, cz))
    assert np.abs(gm - em).max() <= 1e-4 * np.abs(em).max()
    assert np.abs(gz - ez).max() <= 1e-4 * np.abs(ez).max()
    ex.release()


def test_evoformer_block_f16_at_alphafold_widths(dev):
    # f16 at AlphaFold's widths (c_m 256 over 8 heads, c_z 128 over 4; the MFMA
    # flash kernel and the fused kernels), 50 residues and 9 sequences, within
    # 1e-2 of the oracle's largest value.
    import torch

    from afhip.execution import EvoformerBlock, Execution

    L, S, cm, co, cz, ch = 50, 9, 256, 32, 128, 128
    w = _block_weights(0xAF2500, cz, ch, cm, co, 4 * cz)
    w.update(_msa_weights(0xAF2600, cm, cz))
    msa = ref.round_f16(ref.normal(13, (S, L, cm)))
    msa_mask = (ref.uniform(14, (S, L), 0, 1) > 0.1).astype(np.float32)
    pair_mask = (ref.uniform(15, (L, L), 0, 1) > 0.15).astype(np.float32)
    z = ref.round_f16(ref.normal(16, (L, L, cz)))
    em, ez = _oracle_block(msa, msa_mask, z, pair_mask, w, S, L, cm, cz, False)
    ex = Execution()
    blk = EvoformerBlock(ex, L, sequences=S, c_m=cm, c_z=cz, c_outer=co, c_hidden=ch)
    blk.prepare(w)
    tm = torch.from_numpy(msa).half().to(dev)
    tz = torch.from_numpy(z).half().to(dev)
    blk(tm, torch.from_numpy(msa_mask).to(dev), tz, torch.from_numpy(pair_mask).to(dev))
    torch.cuda.synchronize()
    assert np.abs(tm.float().cpu().numpy() - em).max() <= 1e-2 * np.abs(em).max()
    assert np.abs(tz.float().cpu().numpy() - ez).max() <= 1e-2 * np.abs(ez).max()
    ex.release()
