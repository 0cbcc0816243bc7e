"""Per-operation profiling of the Context mirror (KIDI_PROFILE_OPS, ops/context.cpp:117-133, :406-438, :450-455,
:502-515): the aggregation key, request skipping by phase, the report lines; on the GPU, a sync-mode context times
its calls with device events."""

import io

import numpy as np
import pytest
import torch

from kidi_amd.profiling import Profiler, profile_key


def test_key_format():
    """context.cpp:421-429: each extent and attribute followed by a comma, operands separated by ';'."""
    assert profile_key("decode", "packed_linear", [(1, 2048), (8192, 1024), (8192, 16)], [4, 128, 0]) == \
        "phase=decode|op=packed_linear|shapes=[1,2048,];[8192,1024,];[8192,16,]|attrs=4,128,0,"
    assert profile_key("unspecified", "rms_norm", [(3, 64), (64,)], []) == \
        "phase=unspecified|op=rms_norm|shapes=[3,64,];[64,]|attrs="


def test_modes_and_skip():
    assert not Profiler(torch.device("cpu"), {}).active
    assert not Profiler(torch.device("cpu"), {"KIDI_PROFILE_OPS": "yes"}).requested
    p = Profiler(torch.device("cpu"), {"KIDI_PROFILE_OPS": "host", "KIDI_PROFILE_OPS_SKIP": "2"})
    assert p.requested and not p.active and not p.sync
    p.profile_phase("gemma4_request")
    assert not p.active  # request 1 of 2 skipped
    p.profile_phase("decode")
    assert not p.active and p.phase == "decode"  # other phases do not count requests
    p.profile_phase("gemma4_request")
    assert not p.active
    p.profile_phase("gemma4_request")
    assert p.active and p.phase == "gemma4_request"
    assert Profiler(torch.device("cpu"), {"KIDI_PROFILE_OPS": "sync"}).sync


def test_report_lines():
    p = Profiler(torch.device("cpu"), {"KIDI_PROFILE_OPS": "host"})
    p.profile_phase("prefill")
    for _ in range(3):
        with p.call("rms_norm", [(2, 8), (8,)], []) as rec:
            rec["output"] = torch.zeros((2, 8))
    with pytest.raises(RuntimeError):  # a failed call is not counted
        with p.call("rms_norm", [(2, 8), (8,)], []):
            raise RuntimeError("boom")
    p.synchronize()
    lines = p.report()
    assert len(lines) == 2
    assert lines[0].startswith("kidi_op|device=cpu|mode=host|phase=prefill|op=rms_norm|shapes=[2,8,];[8,]|attrs=|calls=3|")
    kv = dict(f.split("=", 1) for f in lines[0].split("|")[1:])
    assert kv["allocations"] == "3" and kv["output_bytes"] == str(3 * 2 * 8 * 4) and kv["device_ns"] == "0"
    assert lines[1].startswith("kidi_op_sync|device=cpu|phase=prefill|calls=1|wait_ns=")
    out = io.StringIO()
    p.close(out)
    p.close(out)  # printed once
    assert out.getvalue().count("kidi_op|") == 1


@pytest.mark.gpu
def test_context_profiles_calls_on_the_gpu(monkeypatch):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd.ops import Context
    from tests.cases import activations, weights

    monkeypatch.setenv("KIDI_PROFILE_OPS", "sync")
    ctx = Context("cuda:0")
    rng = np.random.default_rng(5)
    values, scales, zp, _ = weights(rng, 256, 512, 4, 128)
    v, s = torch.from_numpy(values).cuda(), torch.from_numpy(scales).cuda()
    x = torch.from_numpy(activations(rng, 2, 512)).cuda()
    ctx.profile_phase("decode")
    for _ in range(3):
        ctx.packed_linear(x, v, s, 4, 128)
    ctx.rms_norm(x, torch.ones(512, device="cuda:0"), 1e-6)
    ctx.synchronize()
    lines = ctx.profile_report()
    pl = [l for l in lines if "|op=packed_linear|" in l]
    assert len(pl) == 1
    assert "phase=decode|op=packed_linear|shapes=[2,512,];[256,256,];[256,4,]|attrs=4,128,0,|calls=3|" in pl[0]
    kv = dict(f.split("=", 1) for f in pl[0].split("|")[1:])
    assert int(kv["device_ns"]) > 0 and int(kv["wait_ns"]) > 0 and int(kv["prepare_ns"]) > 0
    assert kv["output_bytes"] == str(3 * 2 * 256 * 4)
    assert any("|op=rms_norm|" in l and "|calls=1|" in l for l in lines)
    assert any(l.startswith("kidi_op_sync|device=cuda:0|phase=decode|calls=1|") for l in lines)
