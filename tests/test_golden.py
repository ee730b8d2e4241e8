"""Committed golden vectors (tests/golden/born_cases.npz, written by
tests/golden/make_golden.py from the float64 oracle).

CPU: the fixture is what the oracle and the host's eager path produce (so a
later change to either shows up as a diff against committed numbers), and the
literal document-id golden of the reference test holds.
GPU: the HIP kernels reproduce the committed outputs and gradients for every
case, in fp32, bf16 and fp16 (forward) and fp32 / bf16 (backward).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import born_oracle as orc
from util import TOL, abi_forward, max_abs, rel_err, z_row_bound

FIXTURE = Path(__file__).resolve().parent / "golden" / "born_cases.npz"
DATA = np.load(FIXTURE)
CASES = sorted({k.split("/")[0] for k in DATA.files if k.endswith("/q")})


def _case(name):
    g = lambda key: DATA[f"{name}/{key}"]  # noqa: E731
    causal, eps, window = g("meta")
    doc = g("doc_ids")
    sc = g("scale")
    return dict(
        q=g("q"), k=g("k"), v=g("v"), do=g("do"), scale=sc,
        kw=dict(is_causal=bool(causal), eps=float(eps), window_size=int(window),
                doc_ids=doc if doc.size else None),
        out=g("out"), z=g("z"), dq=g("dq"), dk=g("dk"), dv=g("dv"), dscale=g("dscale"),
    )


def _scale_arg(sc):
    return sc if sc.size > 1 else float(sc[0])


def test_fixture_lists_every_case():
    assert len(CASES) >= 7
    assert "causal_d64" in CASES and "window_doc_d16" in CASES and "single_token_d8" in CASES


@pytest.mark.parametrize("name", CASES)
def test_inputs_are_bf16_exact(name):
    c = _case(name)
    for key in ("q", "k", "v", "do"):
        t = torch.from_numpy(c[key])
        assert torch.equal(t.to(torch.bfloat16).float(), t), key


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    c = _case(name)
    o, z = orc.forward(c["q"], c["k"], c["v"], _scale_arg(c["scale"]), **c["kw"])
    np.testing.assert_allclose(o, c["out"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(z, c["z"], rtol=1e-6, atol=0)
    grads = orc.backward(c["q"], c["k"], c["v"], _scale_arg(c["scale"]), c["do"], **c["kw"])
    for got, key in zip(grads, ("dq", "dk", "dv", "dscale")):
        np.testing.assert_allclose(got, c[key], rtol=1e-6, atol=1e-7 * max(1.0, np.abs(c[key]).max()))


@pytest.mark.parametrize("name", CASES)
def test_host_eager_path_matches_fixture(name):
    """flash_born_attention on CPU tensors (the reference's eager branch,
    flash_born.py:681-690) in float64, with autograd for the gradients."""
    from quantumdlblocks_amd import flash_born_attention

    c = _case(name)
    q, k, v = (torch.from_numpy(c[x]).double().requires_grad_(True) for x in ("q", "k", "v"))
    sc = torch.from_numpy(c["scale"]).double()
    sc = (sc if sc.numel() > 1 else sc.reshape(())).requires_grad_(True)
    kw = dict(c["kw"])
    if kw["doc_ids"] is not None:
        kw["doc_ids"] = torch.from_numpy(kw["doc_ids"])
    out = flash_born_attention(q, k, v, sc, **kw)
    np.testing.assert_allclose(out.detach().numpy(), c["out"], rtol=1e-6, atol=1e-7)
    out.backward(torch.from_numpy(c["do"]).double())
    for t, key in ((q, "dq"), (k, "dk"), (v, "dv")):
        ref = c[key]
        np.testing.assert_allclose(t.grad.numpy(), ref, rtol=1e-5, atol=1e-6 * max(1.0, np.abs(ref).max()))
    np.testing.assert_allclose(sc.grad.reshape(-1).numpy(), c["dscale"],
                               rtol=1e-4, atol=1e-6 * max(1.0, np.abs(c["dscale"]).max()))


def test_document_ids_literal_golden():
    from quantumdlblocks_amd import compute_document_ids

    got = compute_document_ids(torch.from_numpy(DATA["docids/idx"]), eot_token_id=50256)
    assert got.dtype == torch.int32
    np.testing.assert_array_equal(got.numpy(), DATA["docids/expected"])
    np.testing.assert_array_equal(orc.compute_document_ids(DATA["docids/idx"]), DATA["docids/expected"])


# ----------------------------------------------------------------------------
# GPU: the HIP path against the committed vectors
# ----------------------------------------------------------------------------

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _gpu_run(c, dtype, dev, grads):
    from quantumdlblocks_amd import flash_born_attention

    q, k, v = (torch.from_numpy(c[x]).to(dev, dtype).requires_grad_(grads) for x in ("q", "k", "v"))
    sc = torch.from_numpy(c["scale"]).to(dev)
    sc = (sc if sc.numel() > 1 else sc.reshape(())).requires_grad_(grads)
    kw = dict(c["kw"])
    if kw["doc_ids"] is not None:
        kw["doc_ids"] = torch.from_numpy(kw["doc_ids"]).to(dev)
    out = flash_born_attention(q, k, v, sc, **kw)
    res = {"out": out.detach().double().cpu().numpy()}
    if grads:
        out.backward(torch.from_numpy(c["do"]).to(dev, dtype))
        for t, key in ((q, "dq"), (k, "dk"), (v, "dv")):
            res[key] = t.grad.double().cpu().numpy()
        res["dscale"] = sc.grad.reshape(-1).double().cpu().numpy()
    torch.cuda.synchronize()
    return res


@pytest.mark.gpu
@pytest.mark.parametrize("dt", list(DTYPES))
@pytest.mark.parametrize("name", CASES)
def test_gpu_forward_matches_fixture(cuda_device, name, dt):
    c = _case(name)
    dtype = DTYPES[dt]
    got = _gpu_run(c, dtype, cuda_device, grads=False)["out"]
    err = rel_err(got, c["out"])
    print(f"golden fwd {name} {dt}: rel={err:.3e} maxabs={max_abs(got, c['out']):.3e}", flush=True)
    assert err <= TOL[dtype]
    # Z (sum of weights + eps, the backward's input) through the C ABI, row by
    # row within the rounding bound of the stored weights.  The fixture's
    # inputs are exact in every dtype (bf16-exact values of moderate size).
    D = c["q"].shape[-1]
    if D % 8 == 0:
        q, k, v = (torch.from_numpy(c[x]).to(cuda_device, dtype).contiguous() for x in ("q", "k", "v"))
        kw = c["kw"]
        _, z = abi_forward(q, k, v, c["scale"], kw["is_causal"], kw["eps"], kw["window_size"], kw["doc_ids"])
        mask = orc.visible_mask(c["q"].shape[2], kw["is_causal"], kw["window_size"], kw["doc_ids"])
        bound = z_row_bound(c["q"], c["k"], c["scale"], c["z"], kw["eps"], dtype, mask)
        zerr = np.abs(z.double().cpu().numpy() - c["z"])
        print(f"golden Z {name} {dt}: max err/bound {(zerr / np.maximum(bound, 1e-300)).max():.3f}", flush=True)
        assert np.all(zerr <= bound)


# Gradients that cancel to ~0 are judged against the size of the terms they
# sum (the oracle's backward_magnitudes) instead of their own size.
FLOOR = {"f32": 1e-6, "bf16": 1e-4}


@pytest.mark.gpu
@pytest.mark.parametrize("dt", list(FLOOR))
@pytest.mark.parametrize("name", CASES)
def test_gpu_backward_matches_fixture(cuda_device, name, dt):
    c = _case(name)
    got = _gpu_run(c, DTYPES[dt], cuda_device, grads=True)
    mags = orc.backward_magnitudes(c["q"], c["k"], c["v"], _scale_arg(c["scale"]), c["do"], **c["kw"])
    # bf16 stores O rounded, and the backward forms delta = dO . O from it
    # (flash_born.py:277, 302); the fixture's delta uses the exact O, so the
    # bf16 comparison allows for that rounding through the floor term.
    for key, mag in zip(("dq", "dk", "dv"), mags):
        e_rel = rel_err(got[key], c[key])
        e_floor = max_abs(got[key], c[key]) / max(mag.max(), 1e-30)
        print(f"golden bwd {name} {dt} {key}: rel={e_rel:.3e} floor={e_floor:.3e}", flush=True)
        assert e_rel <= TOL[DTYPES[dt]] or e_floor <= FLOOR[dt], (key, e_rel, e_floor)
    if dt == "f32":
        # dscale = (2/s) eps sum(delta / Z): compare on the scale of its terms.
        z = c["z"].astype(np.float64)
        delta_scale = np.abs(c["out"] * c["do"]).sum(-1)
        sc = c["scale"].astype(np.float64)
        s_h = sc if sc.size > 1 else np.full(c["q"].shape[1], sc[0])
        terms = (2.0 / np.abs(s_h)) * c["kw"]["eps"] * (delta_scale / z).sum(axis=(0, 2))
        bound = terms.sum() if sc.size == 1 else terms
        assert np.all(np.abs(got["dscale"] - c["dscale"]) <= 1e-4 * np.maximum(bound, 1e-30) + 1e-7)
