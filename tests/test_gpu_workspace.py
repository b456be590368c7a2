"""One workspace shared by every entry, through the C ABI.

Every entry that takes a workspace keeps the K splits' counters in its first
TERNOCL_WS_HEADER_BYTES and writes its partials, re-packed weights and MoE
buffers after them.  So a workspace zeroed once serves any sequence of calls:
a prefill GEMM's split-K partials, an M-tiled BITCOS re-pack or a MoE layer
before a split decode GEMV leave its counters at zero, and the GEMV gives the
bits it gives on a fresh workspace.  A counter found above its last value (a
workspace that was never zeroed) resets itself: the split GEMVs give the same
bits on a workspace filled with 0x7f bytes.  Results are compared bit for bit
with the same call on a freshly zeroed workspace, which the parity tests of
each entry check against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth
from tests.gpu_util import dev_dt, dev_raw, host_u16

pytestmark = pytest.mark.gpu

PREFILL = (1024, 14336, 4096)  # (M, K, N): 4 K slices of 128 x 512 tiles
DECODE = (1, 14336, 4096)      # the GEMV's 4 K slices over 128 strips


def _header_zero(ws) -> bool:
    import ternocl_amd as T
    return not ws[:T.WS_HEADER_BYTES].any().item()


def _counters_reset(ws) -> bool:
    """A header filled with 0x7f bytes after split calls: every counter the plan used is
    back at zero, the others untouched (0x7f7f7f7f); none is left at a partial count."""
    import ternocl_amd as T
    import torch
    c = ws[:T.WS_HEADER_BYTES].view(torch.int32).cpu().numpy().view(np.uint32)
    return bool(np.isin(c, (0, 0x7F7F7F7F)).all() and (c == 0).any())


def _int2_operands(seed, M, K, N, bf16):
    g = synth.rng(seed)
    A = synth.activations(g, (M, K), bf16)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias = formats.f32_to_dt(g.standard_normal(N).astype(np.float32) * np.float32(0.1), bf16)
    return dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16), dev_dt(other, bf16), dev_dt(bias, bf16)


def _int2_decode(T, torch, ops, ws):
    dA, dB, dS, dO, dBias = ops
    M, K, N = DECODE
    dC = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
    T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, 5, False, ws=ws)
    torch.cuda.synchronize()
    return host_u16(dC)


@pytest.mark.parametrize("bf16", [False, True])
def test_int2_prefill_then_decode_share_a_workspace(dev, bf16):
    """The prefill GEMM's split-K partials, then the split decode GEMV, on one workspace."""
    import torch
    import ternocl_amd as T
    M, K, N = PREFILL
    dM, dK, dN = DECODE
    assert T.int2_gemm_ws_bytes(M, N, K) > 0 and T.int2_gemm_ws_bytes(dM, dN, dK) > 0
    need = max(T.int2_gemm_ws_bytes(M, N, K), T.int2_gemm_ws_bytes(dM, dN, dK))
    print(f"shared ws int2 prefill {PREFILL} then decode {DECODE} bf16={bf16} ws={need}", flush=True)
    dec = _int2_operands(81, *DECODE, bf16)
    fresh = torch.zeros(need, dtype=torch.uint8, device="cuda")
    want = _int2_decode(T, torch, dec, fresh)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    pA, pB, pS, _, _ = _int2_operands(82, M, K, N, bf16)
    pC = torch.empty((M, N), dtype=pA.dtype, device="cuda")
    for _ in range(2):
        T.int2_fp16_upcvt_gemm(pA, pB, pS, pC, None, None, M, N, K, 0, False, ws=ws)
        torch.cuda.synchronize()
        assert _header_zero(ws), "the prefill split-K wrote into the counters' header"
        got = _int2_decode(T, torch, dec, ws)
        assert np.array_equal(got, want), "the decode GEMV after a prefill on the same workspace differs"
        assert _header_zero(ws), "the decode GEMV left a counter set"


@pytest.mark.parametrize("bf16", [False, True])
def test_int8_prefill_then_decode_share_a_workspace(dev, bf16):
    """The s8 x s2 prefill's split-K partials, then its split decode GEMV (QMODE 0 and 1)."""
    import torch
    import ternocl_amd as T
    M, K, N = PREFILL
    m1 = DECODE[0]
    need = max(T.int2_int8_gemm_ws_bytes(M, N, K), T.int2_int8_gemm_ws_bytes(m1, N, K))
    assert T.int2_int8_gemm_ws_bytes(M, N, K) > 0 and T.int2_int8_gemm_ws_bytes(m1, N, K) > 0
    print(f"shared ws int8 prefill {PREFILL} then decode M=1 bf16={bf16} ws={need}", flush=True)
    dt = torch.bfloat16 if bf16 else torch.float16

    def quant(seed, rows):
        g = synth.rng(seed)
        A = dev_dt(synth.activations(g, (rows, K), bf16), bf16)
        SA = torch.zeros((K // 128, T.ldsa(rows)), dtype=dt, device="cuda")
        Aq = torch.zeros((rows, K), dtype=torch.int8, device="cuda")
        T.quant_a(A, SA, Aq, rows, K)
        B = dev_raw(synth.int2_weights(g, K, N))
        SB = dev_dt(synth.scales(g, K, N, bf16), bf16)
        return A, SA, Aq, B, SB
    dA, dSA, dAq, dB, dSB = quant(91, m1)

    def decode(ws, qmode):
        C = torch.zeros((m1, N), dtype=dt, device="cuda")
        if qmode == 0:
            T.int2_int8_gemm(None, dAq, dSA, dB, dSB, C, None, None, m1, N, K, ws=ws)
        else:
            T.int2_int8_gemm(dA, None, dSA, dB, dSB, C, None, None, m1, N, K, ws=ws)
        torch.cuda.synchronize()
        return host_u16(C)
    fresh = torch.zeros(need, dtype=torch.uint8, device="cuda")
    want = [decode(fresh, 0), decode(fresh, 1)]
    assert np.array_equal(want[0], want[1]), "QMODE 0 and 1 differ"
    pA, pSA, pAq, pB, pSB = quant(92, M)
    pC = torch.empty((M, N), dtype=dt, device="cuda")
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    for qmode in (0, 1):
        T.int2_int8_gemm(None, pAq, pSA, pB, pSB, pC, None, None, M, N, K, ws=ws)
        torch.cuda.synchronize()
        assert _header_zero(ws), "the int8 prefill split-K wrote into the counters' header"
        assert np.array_equal(decode(ws, qmode), want[qmode]), f"QMODE {qmode} decode after a prefill differs"
        assert _header_zero(ws)


def _bitcos_operands(T, torch, seed, K, N, z, bf16, ls):
    g = synth.rng(seed)
    A = synth.activations(g, (1, K), bf16)
    buf, _ = synth.bitcos_weights(g, K, N, z)
    S = synth.scales(g, K, N, bf16)
    dB = dev_raw(buf)
    dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    return dev_dt(A, bf16), dB, dev_dt(S, bf16), dSR


@pytest.mark.parametrize("bf16", [False, True])
def test_bitcos_mt_then_gemv_share_a_workspace(dev, bf16):
    """The M-tiled BITCOS re-pack (after the header), then the split BITCOS GEMV."""
    import torch
    import ternocl_amd as T
    K, N = 5376, 21504
    ls = T.bitcos_pick_ls(1, N, K)
    gws = T.bitcos_gemv_ws_bytes(N, ls)
    assert gws > 0
    need = max(gws, T.bitcos_gemm_mt_ws_bytes(K, N))
    print(f"shared ws bitcos mt then gemv K={K} N={N} ls={ls} bf16={bf16} ws={need}", flush=True)
    A, B, S, SR = _bitcos_operands(T, torch, 93, K, N, 0.5, bf16, ls)
    dt = A.dtype

    def gemv(ws):
        C = torch.zeros((1, N), dtype=dt, device="cuda")
        T.bitcos_fp16_upcvt_gemm(A, B, S, SR, C, None, None, 1, N, K, ls, ws=ws)
        torch.cuda.synchronize()
        return host_u16(C)
    want = gemv(torch.zeros(need, dtype=torch.uint8, device="cuda"))
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    Mp = 64
    Ap = dev_dt(synth.activations(synth.rng(94), (Mp, K), bf16), bf16)
    Cp = torch.empty((Mp, N), dtype=dt, device="cuda")
    T.bitcos_fp16_upcvt_gemm_mt(Ap, B, S, SR, Cp, None, None, Mp, N, K, ls, ws)
    torch.cuda.synchronize()
    assert _header_zero(ws), "the re-pack wrote into the counters' header"
    assert np.array_equal(gemv(ws), want), "the BITCOS GEMV after an M-tiled call on the same workspace differs"
    assert _header_zero(ws)


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_layer_then_decode_share_a_workspace(dev, bf16):
    """A MoE prefill layer's buffers lie after the header: a split GEMV on the same workspace
    afterwards gives its fresh-workspace bits."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I = 64, 8, 2, 256, 256
    need = max(T.int2_moe_prefill_ws_bytes(Tk, E, topk, H, I), T.int2_gemm_ws_bytes(DECODE[0], DECODE[2], DECODE[1]))
    print(f"shared ws moe prefill then decode GEMV bf16={bf16} ws={need}", flush=True)
    dec = _int2_operands(95, *DECODE, bf16)
    want = _int2_decode(T, torch, dec, torch.zeros(need, dtype=torch.uint8, device="cuda"))
    g = synth.rng(96)
    X = dev_dt(synth.activations(g, (Tk, H), bf16), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    W = []
    for K_, N_ in ((H, I), (H, I), (I, H)):
        W.append(dev_raw(np.stack([synth.int2_weights(g, K_, N_) for _ in range(E)])))
        W.append(dev_dt(np.stack([synth.scales(g, K_, N_, bf16) for _ in range(E)]), bf16))
    O = torch.empty((Tk, H), dtype=X.dtype, device="cuda")
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    T.int2_moe_prefill(X, torch.from_numpy(ids).cuda(), dev_dt(RW, bf16), Tk, E, topk, H, I, *W, O, ws)
    torch.cuda.synchronize()
    assert _header_zero(ws), "the MoE layer wrote into the counters' header"
    assert np.array_equal(_int2_decode(T, torch, dec, ws), want)


@pytest.mark.parametrize("bf16", [False, True])
def test_split_gemvs_on_a_workspace_never_zeroed(dev, bf16):
    """Counters reading 0x7f7f7f7f (above every slice count) reset on the first arrival:
    the int2 GEMV, the s8 x s2 GEMV and the BITCOS GEMV give their fresh-workspace bits on
    a workspace filled with 0x7f bytes, and leave its counters at zero."""
    import torch
    import ternocl_amd as T
    print(f"never-zeroed ws: split GEMVs bf16={bf16}", flush=True)
    M, K, N = DECODE
    dec = _int2_operands(97, M, K, N, bf16)
    need = T.int2_gemm_ws_bytes(M, N, K)
    want = _int2_decode(T, torch, dec, torch.zeros(need, dtype=torch.uint8, device="cuda"))
    ws = torch.full((need,), 0x7f, dtype=torch.uint8, device="cuda")
    assert np.array_equal(_int2_decode(T, torch, dec, ws), want), "int2 GEMV on an unzeroed workspace differs"
    assert _counters_reset(ws), "int2 GEMV counters not reset"

    dt = torch.bfloat16 if bf16 else torch.float16
    g = synth.rng(98)
    A = dev_dt(synth.activations(g, (M, K), bf16), bf16)
    SA = torch.zeros((K // 128, T.ldsa(M)), dtype=dt, device="cuda")
    Aq = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    T.quant_a(A, SA, Aq, M, K)
    B, SB = dev_raw(synth.int2_weights(g, K, N)), dev_dt(synth.scales(g, K, N, bf16), bf16)
    need8 = T.int2_int8_gemm_ws_bytes(M, N, K)

    def gemv8(w):
        C = torch.zeros((M, N), dtype=dt, device="cuda")
        T.int2_int8_gemm(None, Aq, SA, B, SB, C, None, None, M, N, K, ws=w)
        torch.cuda.synchronize()
        return host_u16(C)
    want8 = gemv8(torch.zeros(need8, dtype=torch.uint8, device="cuda"))
    ws8 = torch.full((need8,), 0x7f, dtype=torch.uint8, device="cuda")
    assert np.array_equal(gemv8(ws8), want8), "s8 x s2 GEMV on an unzeroed workspace differs"
    assert _counters_reset(ws8), "s8 x s2 GEMV counters not reset"

    Kb, Nb = 5376, 21504
    ls = T.bitcos_pick_ls(1, Nb, Kb)
    Ab, Bb, Sb, SRb = _bitcos_operands(T, torch, 99, Kb, Nb, 0.5, bf16, ls)
    needb = T.bitcos_gemv_ws_bytes(Nb, ls)

    def gemvb(w):
        C = torch.zeros((1, Nb), dtype=dt, device="cuda")
        T.bitcos_fp16_upcvt_gemm(Ab, Bb, Sb, SRb, C, None, None, 1, Nb, Kb, ls, ws=w)
        torch.cuda.synchronize()
        return host_u16(C)
    wantb = gemvb(torch.zeros(needb, dtype=torch.uint8, device="cuda"))
    wsb = torch.full((needb,), 0x7f, dtype=torch.uint8, device="cuda")
    assert np.array_equal(gemvb(wsb), wantb), "BITCOS GEMV on an unzeroed workspace differs"
    assert _counters_reset(wsb), "BITCOS GEMV counters not reset"
