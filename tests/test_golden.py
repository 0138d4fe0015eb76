"""Golden fixtures (tests/golden/golden_v1.npz): the oracle reproduces them bit
for bit on the CPU, and the HIP path matches them within the parity bars on
the GPU.  Crane's repository has no golden vectors for this path; these were
written by tests/golden/make_golden.py from the oracle after a float64 check."""
import json
import os
import sys

import numpy as np
import pytest

from tolerance import assert_close, assert_ulp_close

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from golden_cases import CASES, D, inputs, run_oracle  # noqa: E402

FIXTURE = os.path.join(HERE, "golden", "golden_v1.npz")


def load():
    z = np.load(FIXTURE)   # plain arrays, no pickles
    out = {}
    for name in CASES:
        spec = json.loads(bytes(z[f"{name}.spec"]).decode())
        arrays = {k.split(".", 1)[1]: z[k] for k in z.files if k.startswith(name + ".") and not k.endswith(".spec")}
        out[name] = (spec, arrays)
    return out


GOLDEN = load()


def test_fixture_lists_every_case():
    assert set(GOLDEN) == set(CASES)
    for name, (spec, _) in GOLDEN.items():
        assert spec == json.loads(json.dumps(CASES[name], sort_keys=True)), name


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_reproduces_golden(orc, name):
    spec, want = GOLDEN[name]
    got = run_oracle(orc, spec)
    assert set(got) == set(want)
    for key in want:
        assert np.array_equal(np.asarray(got[key]), want[key]), f"{name}.{key} differs from the fixture"


def test_golden_detects_a_planted_mistake(orc):
    """A wrong sign in the rotate-half RoPE (planted in the oracle's inputs, on
    the CPU) no longer matches the fixture."""
    spec, want = GOLDEN["append_qwen3_f32"]
    x = inputs(orc, spec)
    q = orc.qk_norm_rope_append(x["qkv"], spec["Hq"], spec["Hkv"], x["cos"], -x["sin"], x["positions"],
                                x["k_cache"], x["v_cache"], x["cache_len"], order=spec["order"], dtype="f32")
    assert not np.allclose(q, want["q_out"], atol=1e-3)


# ------------------------------------------------------------------ GPU side

def _dev(x, dtype, gpu):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(gpu).contiguous()


def _host(t):
    return t.float().cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("name", [n for n, s in CASES.items() if s["kind"] in ("append", "decode", "prefill")])
def test_hip_matches_golden(gpu, orc, name):
    import torch
    from crane_amd import ops
    spec, want = GOLDEN[name]
    x = inputs(orc, spec)
    dt = spec["dtype"]
    print(f"golden {name}: {spec}", flush=True)
    i32 = lambda a: torch.as_tensor(np.asarray(a, np.int32), device=gpu)   # noqa: E731
    if spec["kind"] == "append":
        kd, vd = _dev(x["k_cache"], dt, gpu), _dev(x["v_cache"], dt, gpu)
        orders = {0: "norm_then_rope", 1: "rope_then_norm", 2: "rope_only"}
        qw = _dev(x["q_w"], dt, gpu) if x["q_w"] is not None else None
        kw = _dev(x["k_w"], dt, gpu) if x["k_w"] is not None else None
        q = ops.qk_norm_rope_append(_dev(x["qkv"], dt, gpu), _dev(x["cos"], dt, gpu), _dev(x["sin"], dt, gpu),
                                    i32(x["positions"]), kd, vd, i32(x["cache_len"]), spec["cap"], spec["Hq"],
                                    spec["Hkv"], q_norm_w=qw, k_norm_w=kw, order=orders[spec["order"]])
        assert_ulp_close(_host(q), want["q_out"], dt, f"{name} q", min_exact=0.999)
        assert_ulp_close(_host(kd), want["k_cache"], dt, f"{name} k", min_exact=0.999)
        assert np.array_equal(_host(vd), want["v_cache"]), f"{name}: V rows are copied unchanged"
    elif spec["kind"] == "decode":
        out = ops.attention_decode(_dev(x["q"], dt, gpu), _dev(x["k"], dt, gpu), _dev(x["v"], dt, gpu),
                                   i32(x["lens"]), int(max(spec["lens"])))
        assert_close(_host(out).reshape(want["out"].shape), want["out"], dt, name)
    else:
        out = ops.attention_prefill(_dev(x["q"], dt, gpu), _dev(x["k"], dt, gpu), _dev(x["v"], dt, gpu),
                                    i32(x["start"]), int(max(spec["start"])), causal=bool(spec["causal"]))
        assert_close(_host(out).reshape(want["out"].shape), want["out"], dt, name)
