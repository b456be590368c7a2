"""The allocation-free MoE decode entry (ternocl_int2_moe_decode_noalloc), called
through the C ABI: its output equals the workspace entry's
(ternocl_int2_moe_decode) bit for bit, on two calls in a row with the second
smaller than the first (the shared per-device scratch keeps the first call's
contents), for the fused down-and-sum path (topk <= 16) and the path through
the fp32 down rows (topk > 16).  Its host-side size check runs in the CPU
suite (tests/test_abi.py), where no kernel can launch."""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import synth
from tests.gpu_util import dev_dt, dev_raw, host_u16

pytestmark = pytest.mark.gpu


def _case(torch, seed, Tk, E, topk, H, I, bf16):
    g = synth.rng(seed)
    X = dev_dt(synth.activations(g, (Tk, H), bf16), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)

    def experts(K, N):
        return (dev_raw(np.stack([synth.int2_weights(g, K, N) for _ in range(E)])),
                dev_dt(np.stack([synth.scales(g, K, N, bf16) for _ in range(E)]), bf16))
    W = experts(H, I) + experts(H, I) + experts(I, H)
    return X, torch.from_numpy(ids).cuda(), dev_dt(RW, bf16), W


def _run_both(T, torch, case, Tk, E, topk, H, I, bf16):
    L = T.lib()
    X, ids, RW, W = case
    p = [t.data_ptr() for t in W]
    st = torch.cuda.current_stream().cuda_stream
    dt = 1 if bf16 else 0
    O_ws = torch.full((Tk, H), 3.0, dtype=X.dtype, device="cuda")
    O_na = torch.full((Tk, H), 5.0, dtype=X.dtype, device="cuda")
    ws = torch.full((L.ternocl_int2_moe_decode_ws_bytes(Tk, topk, H, I),), 0x7f, dtype=torch.uint8, device="cuda")
    assert L.ternocl_int2_moe_decode(dt, X.data_ptr(), ids.data_ptr(), RW.data_ptr(), Tk, E, topk, H, I, *p,
                                     O_ws.data_ptr(), ws.data_ptr(), ws.numel(), st) == 0
    assert L.ternocl_int2_moe_decode_noalloc(dt, X.data_ptr(), ids.data_ptr(), RW.data_ptr(), Tk, E, topk, H, I,
                                             *p, O_na.data_ptr(), st) == 0, L.ternocl_last_error()
    torch.cuda.synchronize()
    return host_u16(O_ws), host_u16(O_na)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("topk,first,second", [(8, (6, 32, 1024, 768), (1, 16, 512, 256)),
                                              (20, (3, 24, 512, 512), (2, 24, 256, 256))])
def test_noalloc_decode_matches_workspace_entry(dev, bf16, topk, first, second):
    import torch
    import ternocl_amd as T
    for i, (Tk, E, H, I) in enumerate((first, second)):
        print(f"noalloc decode call {i}: T={Tk} E={E} topk={topk} H={H} I={I} bf16={bf16}", flush=True)
        case = _case(torch, 300 + i + topk, Tk, E, topk, H, I, bf16)
        o_ws, o_na = _run_both(T, torch, case, Tk, E, topk, H, I, bf16)
        assert np.array_equal(o_ws, o_na), f"call {i}: the allocation-free entry differs from the workspace entry"

