"""grout_attn_decode_fused_noalloc (static device scratch, no allocation)
against grout_attn_decode_fused (caller scratch) through the C ABI.

Both launch the same kernel on the same inputs, and the kernel's
accumulation order is fixed (each wavefront owns fixed sub-chunks of its
split, the merge walks the splits in order), so q_out, the cache row
written, the merged attention and the advanced position must all be
bit-identical.  Two calls in a row on one GPU, the second with a smaller
input (fewer heads, splits and a shorter context), check that the shared
array's contents from the first call do not leak into the second; a call
whose scratch need exceeds the static array is rejected with
GROUT_ERR_SCRATCH before any launch.  A fresh process checks the first use
of a device: a first call on a stream under capture returns GROUT_ERR_GRAPH
and leaves the capture usable, and the first real call, on a non-default
stream, matches the caller-scratch entry point bit for bit.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from tests._util import (D, EPS, THETA, normal_f16, norm_weight, qk_scale_f16_bits,
                         rng)

pytestmark = pytest.mark.gpu

GROUT_ERR_SCRATCH = -11
GROUT_ERR_GRAPH = -10


def _inputs(torch, seed, hq, hkv, MS, pos):
    g = rng(seed)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    kc = normal_f16(g, (hkv, MS, D))
    vc = normal_f16(g, (hkv, MS, D))
    return dict(qkv=t(normal_f16(g, ((hq + 2 * hkv) * D,))), qw=t(norm_weight(g)),
                kw=t(norm_weight(g)), inv=t(oracle.build_inv_freq(THETA)), kc=kc, vc=vc,
                hq=hq, hkv=hkv, MS=MS, pos=pos)


def _run(torch, L, x, ns, noalloc):
    """One call on fresh copies of the caches; returns the host outputs."""
    import grout_amd

    hq, hkv, G = x["hq"], x["hkv"], x["hq"] // x["hkv"]
    kc = torch.from_numpy(x["kc"]).cuda()
    vc = torch.from_numpy(x["vc"]).cuda()
    q_out = torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda")
    out = torch.full((hkv, G, D), float("nan"), dtype=torch.float16, device="cuda")
    pos = torch.tensor([x["pos"]], dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    common = (x["qkv"].data_ptr(), x["qw"].data_ptr(), x["kw"].data_ptr(), x["inv"].data_ptr(),
              q_out.data_ptr(), kc.data_ptr(), vc.data_ptr())
    tail = (EPS, qk_scale_f16_bits(), hq, hkv, D, x["MS"], 32, ns, 1, st)
    if noalloc:
        status = L.grout_attn_decode_fused_noalloc(*common, out.data_ptr(), pos.data_ptr(), *tail)
    else:
        att, lse = grout_amd.decode_scratch(hkv, G, ns)
        counters = grout_amd.decode_counters(hkv)
        status = L.grout_attn_decode_fused(*common, att.data_ptr(), lse.data_ptr(),
                                           out.data_ptr(), counters.data_ptr(), pos.data_ptr(),
                                           *tail)
    assert status == 0, f"status {status}"
    torch.cuda.synchronize()
    return dict(out=out.cpu().numpy(), q_out=q_out.cpu().numpy(), kc=kc.cpu().numpy(),
                vc=vc.cpu().numpy(), pos=int(pos.item()))


def _same(a, b, what):
    for k in ("q_out", "kc", "vc"):
        assert np.array_equal(a[k].view(np.uint16), b[k].view(np.uint16)), f"{what}: {k} differs"
    assert np.array_equal(a["out"].view(np.uint16), b["out"].view(np.uint16)), f"{what}: out differs"
    assert a["pos"] == b["pos"], f"{what}: position {a['pos']} != {b['pos']}"


def test_noalloc_matches_caller_scratch_twice(gpu):
    import torch

    import grout_amd

    L = grout_amd.lib()
    big = _inputs(torch, 900, 64, 8, 33000, 32768)    # c4 shapes, 32 splits
    small = _inputs(torch, 901, 32, 4, 5000, 4096)     # fewer heads, splits, keys
    cases = ((big, 32), (small, 12))
    print("[noalloc] two calls in a row: c4 shapes, then 32/4 heads ctx 4096", flush=True)
    got = [_run(torch, L, x, ns, noalloc=True) for x, ns in cases]
    ref = [_run(torch, L, x, ns, noalloc=False) for x, ns in cases]
    for (x, _), a, b in zip(cases, got, ref):
        _same(a, b, f"{x['hq']}/{x['hkv']} heads")
        assert a["pos"] == x["pos"] + 1
        assert np.isfinite(a["out"].astype(np.float32)).all()


def test_noalloc_rejects_beyond_static_scratch(gpu):
    import torch

    import grout_amd

    L = grout_amd.lib()
    x = _inputs(torch, 902, 64, 8, 2048, 1000)
    out = torch.zeros((8, 8, D), dtype=torch.float16, device="cuda")
    q_out = torch.zeros((72, D), dtype=torch.float16, device="cuda")
    kc = torch.from_numpy(x["kc"]).cuda()
    vc = torch.from_numpy(x["vc"]).cuda()
    pos = torch.tensor([1000], dtype=torch.int32, device="cuda")
    before = kc.clone()
    args = lambda ns, hkv_lim=8: (  # noqa: E731
        x["qkv"].data_ptr(), x["qw"].data_ptr(), x["kw"].data_ptr(), x["inv"].data_ptr(),
        q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), pos.data_ptr(), EPS,
        qk_scale_f16_bits(), 64, hkv_lim, D, 2048, 32, ns, 1, 0)
    # 64 heads x 256 splits = 16384 rows of 260 B > 4 MiB - 64 KiB.
    assert L.grout_attn_decode_fused_noalloc(*args(256)) == GROUT_ERR_SCRATCH
    assert L.grout_attn_decode_fused_noalloc(*args(1025)) == -8   # GROUT_ERR_SPLITS
    torch.cuda.synchronize()
    assert torch.equal(before, kc) and int(pos.item()) == 1000, "a rejected call launched"
    assert "static scratch" in L.grout_status_string(GROUT_ERR_SCRATCH).decode()


# Run in a child process, so that its calls are the first on the device.
_FIRST_USE = r"""
import json, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
import grout_amd
from tests import test_zz_no_alloc as t

L = grout_amd.lib()
x = t._inputs(torch, 903, 32, 8, 4200, 4096)
side = torch.cuda.Stream()
res = {}
with torch.cuda.stream(side):
    kc = torch.from_numpy(x["kc"]).cuda()
    vc = torch.from_numpy(x["vc"]).cuda()
    q_out = torch.zeros((40, t.D), dtype=torch.float16, device="cuda")
    out = torch.zeros((8, 4, t.D), dtype=torch.float16, device="cuda")
    pos = torch.tensor([4096], dtype=torch.int32, device="cuda")
    flag = torch.zeros((1,), dtype=torch.int32, device="cuda")
torch.cuda.synchronize()
st = side.cuda_stream
args = (x["qkv"].data_ptr(), x["qw"].data_ptr(), x["kw"].data_ptr(), x["inv"].data_ptr(),
        q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), pos.data_ptr(),
        t.EPS, t.qk_scale_f16_bits(), 32, 8, t.D, 4200, 32, 16, 1, st)
# First call of the process, on a stream under capture: refused, and the
# capture goes on (a kernel recorded after it runs when the graph replays).
import ctypes
assert L.grout_graph_begin(st) == 0
res["capture_status"] = int(L.grout_attn_decode_fused_noalloc(*args))
res["record_status"] = int(L.grout_set_position_async(flag.data_ptr(), 7, st))
g = ctypes.c_void_p()
res["end_status"] = int(L.grout_graph_end(st, ctypes.byref(g)))
res["launch_status"] = int(L.grout_graph_launch(g, st))
side.synchronize()
res["flag"] = int(flag.item())
L.grout_graph_destroy(g)
# First real call: on the side stream.
res["call_status"] = int(L.grout_attn_decode_fused_noalloc(*args))
side.synchronize()
ref = t._run(torch, L, x, 16, noalloc=False)
res["out_equal"] = bool(np.array_equal(out.cpu().numpy().view(np.uint16), ref["out"].view(np.uint16)))
res["kc_equal"] = bool(np.array_equal(kc.cpu().numpy().view(np.uint16), ref["kc"].view(np.uint16)))
res["pos"] = int(pos.item())
print("RESULT " + json.dumps(res), flush=True)
"""


def test_noalloc_first_use_in_fresh_process(gpu):
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[noalloc] fresh process: first call under capture, then on a side stream", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_USE, root], cwd=root, capture_output=True,
                       text=True, timeout=300)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("RESULT ")]
    assert r.returncode == 0 and lines, f"child failed (rc {r.returncode}):\n{r.stdout}\n{r.stderr}"
    res = json.loads(lines[-1][len("RESULT "):])
    assert res["capture_status"] == GROUT_ERR_GRAPH, res
    assert res["record_status"] == 0 and res["end_status"] == 0 and res["launch_status"] == 0, res
    assert res["flag"] == 7, res
    assert res["call_status"] == 0, res
    assert res["out_equal"] and res["kc_equal"], res
    assert res["pos"] == 4097, res
