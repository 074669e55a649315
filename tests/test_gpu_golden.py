"""GPU kernels against the committed golden fixtures (no oracle call): V and
KV slots bit-exact, Q/K within 1 f16 ulp, attention within 2e-3 + 1e-2|ref|."""
import math
import os

import numpy as np
import pytest

from tests._util import assert_close_attn, f16_ulp_diff

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D = 128


def load(name):
    return np.load(os.path.join(GOLD, name))


def dev(torch, bits_or_f32):
    a = np.ascontiguousarray(bits_or_f32)
    if a.dtype == np.uint16:
        a = a.view(np.float16)
    return torch.from_numpy(a.copy()).cuda()


def test_norm_rope_prefill_golden(gpu):
    import torch

    import grout_amd

    z = load("qk_norm_rope_prefill.npz")
    q, k, v = dev(torch, z["q"]), dev(torch, z["k"]), dev(torch, z["v"])
    kc = torch.zeros_like(dev(torch, z["k_cache"]))
    vc = torch.zeros_like(kc)
    qo = torch.zeros_like(q)
    grout_amd.qk_norm_rope_kv_prefill(q, k, v, dev(torch, z["q_weight"]), dev(torch, z["k_weight"]),
                                      dev(torch, z["inv_freq"]), qo, kc, vc, float(z["eps"]),
                                      int(z["position_start"]))
    torch.cuda.synchronize()
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), z["v_cache"])
    assert f16_ulp_diff(qo.cpu().numpy(), z["q_out"].view(np.float16)).max() <= 1
    assert f16_ulp_diff(kc.cpu().numpy(), z["k_cache"].view(np.float16)).max() <= 1


def test_norm_rope_decode_golden(gpu):
    import torch

    import grout_amd

    z = load("qk_norm_rope_decode.npz")
    hkv = z["k_cache_in"].shape[0]
    hq = z["q_out"].shape[0] - hkv
    kc, vc = dev(torch, z["k_cache_in"]), dev(torch, z["v_cache_in"])
    qo = torch.zeros((hq + hkv, D), dtype=torch.float16, device="cuda")
    pos = torch.tensor([int(z["position"])], dtype=torch.int32, device="cuda")
    grout_amd.qk_norm_rope_kv_decode(dev(torch, z["qkv"]), dev(torch, z["q_weight"]),
                                     dev(torch, z["k_weight"]), dev(torch, z["inv_freq"]), qo, kc,
                                     vc, pos, float(z["eps"]), hq, hkv)
    torch.cuda.synchronize()
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), z["v_cache"])
    assert f16_ulp_diff(qo.cpu().numpy(), z["q_out"].view(np.float16)).max() <= 1
    assert f16_ulp_diff(kc.cpu().numpy(), z["k_cache"].view(np.float16)).max() <= 1


def test_attn_prefill_golden(gpu):
    import torch

    import grout_amd

    z = load("attn_prefill.npz")
    for key in ("S17_qs0", "S17_qs5", "S64_qs0", "S64_qs5"):
        qs = int(key.split("qs")[1])
        q = dev(torch, z[key + "_q"])
        out = torch.empty_like(q)
        grout_amd.attend_prefill(q, dev(torch, z[key + "_k"]), dev(torch, z[key + "_v"]), out, qs)
        torch.cuda.synchronize()
        assert_close_attn(out.cpu().numpy(), z[key + "_out"], key)


def test_attn_decode_golden(gpu):
    import torch

    import grout_amd

    z = load("attn_decode.npz")
    q = dev(torch, z["q"])
    hkv, G, _ = q.shape
    pos = torch.tensor([int(z["position"])], dtype=torch.int32, device="cuda")
    for ns in (1, 3):
        att, lse = grout_amd.decode_scratch(hkv, G, ns)
        grout_amd.fmha_decode_gqa_split(q, dev(torch, z["k_cache"]), dev(torch, z["v_cache"]), att,
                                        lse, int(z["qk_scale_f16"]), pos, int(z["block_n"]))
        out = torch.empty((hkv, G, D), dtype=torch.float16, device="cuda")
        grout_amd.splitk_reduce_merge(att, lse, out)
        torch.cuda.synchronize()
        assert_close_attn(att.cpu().numpy(), z[f"nks{ns}_att"].view(np.float16), f"att nks={ns}")
        assert np.max(np.abs(lse.cpu().numpy() - z[f"nks{ns}_lse"])) < 1e-3
        assert_close_attn(out.cpu().numpy(), z[f"nks{ns}_out"].view(np.float16), f"out nks={ns}")
