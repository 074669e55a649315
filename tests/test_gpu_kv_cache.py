"""GPU parity of the KV-cache suffix writer (kv_cache_update_seq_f16 and its
device-position form) against the oracle and the reference's own KAT."""
import numpy as np
import pytest

import oracle
from tests._util import normal_f16, rng

pytestmark = pytest.mark.gpu


def test_reference_kat_on_gpu(gpu):
    """tests/kernels.rs:67-118 on the GPU: D=4, 2 heads, capacity 16, 5 rows at 3."""
    import torch

    import grout_amd

    HEADS, CAP, D, ROWS, START = 2, 16, 4, 5, 3
    values = (np.arange(ROWS * HEADS * D) + 1).astype(np.float16).reshape(ROWS, HEADS, D)
    dv = torch.from_numpy(values).cuda()
    k = torch.zeros((HEADS, CAP, D), dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    grout_amd.kv_cache_update_seq(dv, dv, k, v, START)
    torch.cuda.synchronize()
    k_ref = np.zeros((HEADS, CAP, D), np.float16)
    v_ref = np.zeros((HEADS, CAP, D), np.float16)
    oracle.kv_cache_update_seq(values, values, k_ref, v_ref, START)
    assert np.array_equal(k.cpu().numpy().view(np.uint16), k_ref.view(np.uint16))
    assert np.array_equal(v.cpu().numpy().view(np.uint16), v_ref.view(np.uint16))


@pytest.mark.parametrize("hkv,MS,S,start,seed", [
    (8, 300, 50, 37, 1),       # unaligned nonzero start (MTP suffix)
    (8, 4200, 1, 4096, 2),     # one row (decode position of config c2)
    (2, 64, 64, 0, 3),         # whole cache
])
def test_update_matches_oracle(gpu, hkv, MS, S, start, seed):
    import torch

    import grout_amd

    g = rng(seed)
    D = 128
    nk, nv = normal_f16(g, (S, hkv, D)), normal_f16(g, (S, hkv, D))
    kc = np.full((hkv, MS, D), 7.0, np.float16)
    vc = np.full((hkv, MS, D), -3.0, np.float16)
    dk, dv = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    grout_amd.kv_cache_update_seq(torch.from_numpy(nk).cuda(), torch.from_numpy(nv).cuda(), dk,
                                  dv, start)
    torch.cuda.synchronize()
    oracle.kv_cache_update_seq(nk, nv, kc, vc, start)
    assert np.array_equal(dk.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(dv.cpu().numpy().view(np.uint16), vc.view(np.uint16))


@pytest.mark.parametrize("hkv,D,MS,S,start,seed", [
    (3, 64, 100, 37, 5, 11),     # odd head count, 8 16-byte units per row, ragged last tile
    (1, 12, 40, 17, 2, 12),      # 8-byte units (head_dim % 8 != 0), 3 per row
    (5, 8, 33, 33, 0, 13),       # one unit per row, the whole cache
    (4, 256, 70, 19, 51, 14),    # 32 units per row, the last row written is the cache's last
    (7, 128, 5000, 4099, 901, 15),  # many tiles, the last one 3 rows
])
def test_update_head_dims_and_tiles(gpu, hkv, D, MS, S, start, seed):
    """The writer's 16-token tiles over every lane layout it supports: head_dim a
    multiple of 4 (16- or 8-byte units), any head count, seq_len not a multiple
    of the tile, a sentinel everywhere else in the caches."""
    import torch

    import grout_amd

    g = rng(seed)
    nk, nv = normal_f16(g, (S, hkv, D)), normal_f16(g, (S, hkv, D))
    kc = np.full((hkv, MS, D), 7.0, np.float16)
    vc = np.full((hkv, MS, D), -3.0, np.float16)
    dk, dv = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    grout_amd.kv_cache_update_seq(torch.from_numpy(nk).cuda(), torch.from_numpy(nv).cuda(), dk,
                                  dv, start)
    torch.cuda.synchronize()
    oracle.kv_cache_update_seq(nk, nv, kc, vc, start)
    assert np.array_equal(dk.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(dv.cpu().numpy().view(np.uint16), vc.view(np.uint16))


@pytest.mark.parametrize("pos,S", [(60, 20), (0, 33), (79, 1), (80, 17)])
def test_dynpos_rows_past_the_cache_end(gpu, pos, S):
    """The device-position form with several rows (the C entry point; the Python
    mirror keeps the decode path's one row): rows whose slot falls at or past
    max_seq_len are skipped, the others land as the oracle puts them."""
    import torch

    import grout_amd

    g = rng(100 + pos + S)
    hkv, MS, D = 3, 80, 128
    nk, nv = normal_f16(g, (S, hkv, D)), normal_f16(g, (S, hkv, D))
    kc = np.full((hkv, MS, D), 7.0, np.float16)
    vc = np.full((hkv, MS, D), -3.0, np.float16)
    dk, dv = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    tk, tv = torch.from_numpy(nk).cuda(), torch.from_numpy(nv).cuda()
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert grout_amd.lib().grout_kv_cache_update_seq_dynpos(
        tk.data_ptr(), tv.data_ptr(), dk.data_ptr(), dv.data_ptr(), dpos.data_ptr(), S, hkv, D,
        MS, st) == 0
    torch.cuda.synchronize()
    keep = max(0, min(S, MS - pos))
    if keep:
        oracle.kv_cache_update_seq(nk[:keep].copy(), nv[:keep].copy(), kc, vc, pos)
    assert np.array_equal(dk.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(dv.cpu().numpy().view(np.uint16), vc.view(np.uint16))


def test_dynpos_graph_replay_and_guard(gpu):
    """The device-position form captured once in a hipGraph and replayed at three
    positions (set with grout_set_position_async); a position past the cache
    writes nothing."""
    import torch

    import grout_amd
    from grout_amd import _lib

    g = rng(9)
    hkv, MS, D = 8, 96, 128
    L = grout_amd.lib()
    kc = torch.zeros((hkv, MS, D), dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    nk = torch.empty((1, hkv, D), dtype=torch.float16, device="cuda")
    nv = torch.empty_like(nk)
    pos = torch.zeros((1,), dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    k_ref = np.zeros((hkv, MS, D), np.float16)
    v_ref = np.zeros((hkv, MS, D), np.float16)
    with torch.cuda.stream(s):
        assert L.grout_graph_begin(s.cuda_stream) == 0
        grout_amd.kv_cache_update_seq_dynpos(nk, nv, kc, vc, pos)
        graph = _lib.ctypes.c_void_p()
        assert L.grout_graph_end(s.cuda_stream, _lib.ctypes.byref(graph)) == 0
    try:
        for p in (5, 95, 40, 96):
            a, b = normal_f16(g, (1, hkv, D)), normal_f16(g, (1, hkv, D))
            with torch.cuda.stream(s):
                nk.copy_(torch.from_numpy(a).cuda())
                nv.copy_(torch.from_numpy(b).cuda())
                assert L.grout_set_position_async(pos.data_ptr(), p, s.cuda_stream) == 0
                assert L.grout_graph_launch(graph, s.cuda_stream) == 0
            s.synchronize()
            if p < MS:
                oracle.kv_cache_update_seq(a, b, k_ref, v_ref, p)
            assert np.array_equal(kc.cpu().numpy().view(np.uint16), k_ref.view(np.uint16)), p
            assert np.array_equal(vc.cpu().numpy().view(np.uint16), v_ref.view(np.uint16)), p
    finally:
        L.grout_graph_destroy(graph)


def test_python_mirror_errors(gpu):
    import torch

    import grout_amd

    h = torch.float16
    kc = torch.zeros((2, 16, 128), dtype=h, device="cuda")
    nk = torch.zeros((4, 2, 128), dtype=h, device="cuda")
    with pytest.raises(grout_amd.GroutError, match="exceeds max_seq_len"):
        grout_amd.kv_cache_update_seq(nk, nk, kc, kc, 13)
    with pytest.raises(grout_amd.GroutError, match="new_v shape mismatch"):
        grout_amd.kv_cache_update_seq(nk, nk[:3], kc, kc, 0)
    with pytest.raises(grout_amd.GroutError, match="rank 3"):
        grout_amd.kv_cache_update_seq(nk[0], nk[0], kc, kc, 0)
    with pytest.raises(grout_amd.GroutError, match="expects seq_len=1"):
        grout_amd.kv_cache_update_seq_dynpos(nk, nk, kc, kc,
                                             torch.zeros((1,), dtype=torch.int32, device="cuda"))
