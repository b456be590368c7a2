"""The PyTorch custom operators (torch.ops.ternocl.*): registration and shape
propagation on the CPU (meta tensors reach the fake implementations, no
library call), and on the GPU the same bits as the direct C-ABI calls plus
torch.library.opcheck's schema / fake-tensor checks."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")


def test_ops_registered_and_fake_shapes():
    import ternocl_amd.torch_ops  # noqa: F401  (registers the operators)
    ops = torch.ops.ternocl
    M, K, N, E, topk, H, I = 5, 256, 48, 4, 2, 256, 128
    A = torch.empty((M, K), dtype=torch.bfloat16, device="meta")
    B = torch.empty((K // 16, N), dtype=torch.int32, device="meta")
    S = torch.empty((K // 128, N), dtype=torch.bfloat16, device="meta")
    assert ops.int2_gemm(A, B, S, None, None, 0, False).shape == (M, N)
    assert ops.int2_gemm(A, B, S, None, None, 3, True).dtype == torch.float32
    SA, Aq = ops.quant_a(A)
    assert SA.shape == (K // 128, 32) and Aq.shape == (M, K) and Aq.dtype == torch.int8
    assert ops.int2_int8_gemm(Aq, SA, B, S, None, None, 0, False).shape == (M, N)
    Bc = torch.empty(K // 32 * N + N + 64, dtype=torch.int32, device="meta")
    assert ops.bitcos_gemm(A, Bc, S, None, 1, N, None, None, 0, False).shape == (M, N)
    x = torch.empty((2, 1024), dtype=torch.float16, device="meta")
    assert ops.fwht(x, None, 512).shape == x.shape
    X = torch.empty((M, H), dtype=torch.bfloat16, device="meta")
    ids = torch.empty((M, topk), dtype=torch.int32, device="meta")
    RW = torch.empty((M, topk), dtype=torch.bfloat16, device="meta")
    Bg = torch.empty((E, H // 16, I), dtype=torch.int32, device="meta")
    Sg = torch.empty((E, H // 128, I), dtype=torch.bfloat16, device="meta")
    Bd = torch.empty((E, I // 16, H), dtype=torch.int32, device="meta")
    Sd = torch.empty((E, I // 128, H), dtype=torch.bfloat16, device="meta")
    assert ops.moe_prefill(X, ids, RW, E, Bg, Sg, Bg, Sg, Bd, Sd).shape == (M, H)
    assert ops.moe_decode(X, ids, RW, E, Bg, Sg, Bg, Sg, Bd, Sd).shape == (M, H)
    assert ops.moe_prefill_int8(X, ids, RW, E, Bg, Sg, Bg, Sg, Bd, Sd).shape == (M, H)


def test_ops_reject_bad_inputs():
    """Each operator checks dtype, shape and contiguity before any launch (meta
    tensors: the checks run in the fake implementations, no library call)."""
    import ternocl_amd.torch_ops  # noqa: F401
    ops = torch.ops.ternocl
    m = dict(device="meta")
    M, K, N, E, topk, H, I = 5, 256, 48, 4, 2, 256, 128
    A = torch.empty((M, K), dtype=torch.bfloat16, **m)
    B = torch.empty((K // 16, N), dtype=torch.int32, **m)
    S = torch.empty((K // 128, N), dtype=torch.bfloat16, **m)

    def bad(fn, *args):
        with pytest.raises(RuntimeError):
            fn(*args)
    bad(ops.int2_gemm, A.float(), B, S, None, None, 0, False)                 # fp32 activations
    bad(ops.int2_gemm, A, B.long(), S, None, None, 0, False)                   # int64 weights
    bad(ops.int2_gemm, A, B, S.half(), None, None, 0, False)                   # S dtype != A dtype
    bad(ops.int2_gemm, A, B[:, :32], S, None, None, 0, False)                  # S columns != B columns
    bad(ops.int2_gemm, A, B, S, torch.empty((M, N + 16), dtype=A.dtype, **m), None, 2, False)
    bad(ops.int2_gemm, A, B, S, None, torch.empty(N, dtype=A.dtype, **m), 3, True)  # fp32 out: fp32 bias
    bad(ops.int2_gemm, torch.empty((K, M), dtype=A.dtype, **m).t(), B, S, None, None, 0, False)  # not contiguous
    Aq = torch.empty((M, K), dtype=torch.int8, **m)
    SA = torch.empty((K // 128, 32), dtype=torch.bfloat16, **m)
    bad(ops.int2_int8_gemm, Aq, SA[:, :16], B, S, None, None, 0, False)      # SA pitch != ldsa(M)
    bad(ops.int2_int8_gemm, Aq.to(torch.uint8), SA, B, S, None, None, 0, False)
    Bc = torch.empty(K // 32 * N + N + 64, dtype=torch.int32, **m)
    bad(ops.bitcos_gemm, A, Bc, S, None, 2, N, None, None, 0, False)         # ls > 1 needs SR
    bad(ops.fwht, A, torch.empty(K, dtype=torch.float16, **m), 256)           # signs must be int8
    X = torch.empty((M, H), dtype=torch.bfloat16, **m)
    ids = torch.empty((M, topk), dtype=torch.int32, **m)
    RW = torch.empty((M, topk), dtype=torch.bfloat16, **m)
    Bg = torch.empty((E, H // 16, I), dtype=torch.int32, **m)
    Sg = torch.empty((E, H // 128, I), dtype=torch.bfloat16, **m)
    Bd = torch.empty((E, I // 16, H), dtype=torch.int32, **m)
    Sd = torch.empty((E, I // 128, H), dtype=torch.bfloat16, **m)
    for op in (ops.moe_prefill, ops.moe_decode, ops.moe_prefill_int8):
        op(X, ids, RW, E, Bg, Sg, Bg, Sg, Bd, Sd)                               # the good case
        bad(op, X, ids.long(), RW, E, Bg, Sg, Bg, Sg, Bd, Sd)                  # torch.topk's int64 ids
        bad(op, X, ids, RW, E + 1, Bg, Sg, Bg, Sg, Bd, Sd)                     # E != stacked experts
        bad(op, X, ids, RW.half(), E, Bg, Sg, Bg, Sg, Bd, Sd)                  # RW dtype != X dtype
        bad(op, X, ids, RW, E, Bg, Sg, Bg, Sg, Bg, Sd)                         # down weights transposed
        bad(op, X, ids, RW, E, Bg, Sg[:, :, :64], Bg, Sg, Bd, Sd)              # scale shape


@pytest.mark.gpu
def test_ops_match_direct_calls(dev, orc):
    import ternocl_amd as T
    import ternocl_amd.torch_ops  # noqa: F401
    from ternocl_amd import formats, synth
    from tests.gpu_util import dev_dt, dev_raw, host_u16
    ops = torch.ops.ternocl
    g = synth.rng(123)
    M, K, N, bf16 = 3, 1024, 272, True
    A = dev_dt(synth.activations(g, (M, K), bf16), bf16)
    B = dev_raw(synth.int2_weights(g, K, N))
    S = dev_dt(synth.scales(g, K, N, bf16), bf16)
    O = dev_dt(synth.activations(g, (M, N), bf16), bf16)
    bias = dev_dt(formats.f32_to_dt(g.standard_normal(N).astype(np.float32), bf16), bf16)
    C = ops.int2_gemm(A, B, S, O, bias, 5, False)
    C2 = torch.empty_like(C)
    T.int2_fp16_upcvt_gemm(A, B, S, C2, O, bias, M, N, K, 5, False)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(C), host_u16(C2))
    torch.library.opcheck(ops.int2_gemm.default, (A, B, S, O, bias, 5, False),
                          test_utils=("test_schema", "test_faketensor"))

    A16 = dev_dt(synth.activations(g, (64, K), False), False)
    SA, Aq = ops.quant_a(A16)
    S16 = dev_dt(synth.scales(g, K, N, False), False)
    C8 = ops.int2_int8_gemm(Aq, SA, B, S16, None, None, 0, False)
    SA2 = torch.empty_like(SA)
    Aq2 = torch.empty_like(Aq)
    T.quant_a(A16, SA2, Aq2, 64, K)
    C82 = torch.empty_like(C8)
    T.int2_int8_gemm(None, Aq2, SA2, B, S16, C82, None, None, 64, N, K)
    torch.cuda.synchronize()
    assert torch.equal(Aq, Aq2) and np.array_equal(host_u16(C8), host_u16(C82))

    codes = synth.ternary_codes(g, K, N, 0.5)
    buf = dev_raw(formats.bitcos_pack(codes))
    for Mb in (2, 32):
        Ab = dev_dt(synth.activations(g, (Mb, K), False), False)
        Cb = ops.bitcos_gemm(Ab, buf, S16, None, 1, N, None, None, 0, False)
        want = formats.dt_to_f32(orc.epilogue(orc.bitcos_gold(host_u16(Ab), formats.bitcos_pack(codes),
                                                              host_u16(S16), Mb, K, N, False),
                                              None, None, 0, False, False), False)
        got = formats.dt_to_f32(host_u16(Cb), False)
        assert np.all(np.abs(got - want) <= 1e-3 + 1e-2 * np.abs(want))

    x = dev_dt(synth.activations(g, (2, 1024), False), False)
    y = ops.fwht(x, None, 512)
    y2 = torch.empty_like(x)
    T.hadamard_fwht(x, None, y2, 2, 1024, 512, False)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


@pytest.mark.gpu
@pytest.mark.parametrize("Tk,decode", [(40, False), (3, True), (40, "int8")])
def test_moe_ops_match_direct_calls(dev, Tk, decode):
    """moe_prefill / moe_decode / moe_prefill_int8 give the direct C-ABI calls' bits."""
    import numpy as np
    import ternocl_amd as T
    import ternocl_amd.torch_ops  # noqa: F401
    from ternocl_amd import synth
    from tests.gpu_util import dev_dt, dev_raw, host_u16
    E, topk, H, I, bf16 = 6, 2, 256, 128, True
    g = synth.rng(91 + Tk)
    X = dev_dt(synth.activations(g, (Tk, H), bf16), bf16)
    ids_np, RW_np = synth.moe_routing(g, Tk, E, topk, bf16)
    ids = torch.from_numpy(ids_np.reshape(Tk, topk)).cuda()
    RW = dev_dt(RW_np.reshape(Tk, topk), bf16)

    def experts(K, N):
        return (dev_raw(np.stack([synth.int2_weights(g, K, N) for _ in range(E)])),
                dev_dt(np.stack([synth.scales(g, K, N, bf16) for _ in range(E)]), bf16))
    (Bg, Sg), (Bu, Su), (Bd, Sd) = experts(H, I), experts(H, I), experts(I, H)
    op = {False: torch.ops.ternocl.moe_prefill, True: torch.ops.ternocl.moe_decode,
          "int8": torch.ops.ternocl.moe_prefill_int8}[decode]
    got = op(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd)
    O = torch.empty_like(X)
    if decode == "int8":
        ws = torch.empty(T.int2_moe_prefill_int8_ws_bytes(Tk, E, topk, H, I), dtype=torch.uint8, device="cuda")
        T.int2_moe_prefill_int8(X, ids, RW, Tk, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws)
    elif decode:
        ws = torch.empty(T.int2_moe_decode_ws_bytes(Tk, topk, H, I), dtype=torch.uint8, device="cuda")
        T.int2_moe_decode(X, ids, RW, Tk, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws)
    else:
        ws = torch.empty(T.int2_moe_prefill_ws_bytes(Tk, E, topk, H, I), dtype=torch.uint8, device="cuda")
        T.int2_moe_prefill(X, ids, RW, Tk, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(got), host_u16(O))
