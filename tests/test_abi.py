"""The C ABI without a GPU: the header declares exactly the exported symbol
table, the built library exports every symbol, and host-side argument checks
return their status codes before any launch (int2_fp16_upcvt/main.cpp:159 is
the reference's shape check, which exits instead)."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ternocl_amd.h"


def _declared():
    text = HEADER.read_text()
    return set(re.findall(r"\b(ternocl_[a-z0-9_]+)\s*\(", text))


def test_header_matches_symbol_table():
    from ternocl_amd import _abi
    assert _declared() == set(_abi.SYMBOLS), _declared() ^ set(_abi.SYMBOLS)


def test_library_exports_every_declared_symbol():
    import ternocl_amd as T
    path = T.library_path()
    assert path.exists(), "build the library first (python -m ternocl_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (ternocl_[a-z0-9_]+)", out))
    missing = _declared() - exported
    assert not missing, missing
    T.lib()  # loads and binds every signature


def test_header_compiles_as_c():
    src = f'#include "{HEADER}"\nint main(void){{return TERNOCL_OK;}}\n'
    r = subprocess.run(["gcc", "-x", "c", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def _call_gemm(L, **kw):
    a = dict(dtype=0, A=1, B=1, S=1, C=1, Other=None, Bias=None, M=1, N=4096, K=4096,
             postop=0, out_f32=0, ws=None, ws_bytes=0, stream=None)
    a.update(kw)
    return L.ternocl_int2_fp16_upcvt_gemm(*a.values())


@pytest.mark.parametrize("kw,status", [
    (dict(N=4100), 2), (dict(K=4000), 2), (dict(M=0), 2), (dict(dtype=7), 1),
    (dict(A=None), 1), (dict(postop=6), 1), (dict(postop=1), 1), (dict(postop=3), 1),
    (dict(out_f32=2), 1)])
def test_host_validation(kw, status):
    import ternocl_amd as T
    L = T.lib()
    assert _call_gemm(L, **kw) == status
    assert L.ternocl_last_error().decode()


def test_status_strings():
    import ternocl_amd as T
    L = T.lib()
    assert L.ternocl_status_string(0) == b"ok"
    assert L.ternocl_version().decode().count(".") == 2


def test_ws_bytes_query():
    import ternocl_amd as T
    H = T.WS_HEADER_BYTES
    # the fp8 x fp4 GEMV's K split: the 64 KiB workspace header (strip counters) + slices of fp32 [M, N]
    assert T.int2_gemm_ws_bytes(1, 14336, 4096) == 0  # 448 32-column strips fill the chip unsplit
    assert T.int2_gemm_ws_bytes(1, 4096, 14336) == H + 4 * 1 * 4096 * 4  # 128 strips x 4 slices
    assert T.int2_gemm_ws_bytes(8, 4096, 14336) == H + 4 * 8 * 4096 * 4  # 64 strips x 4 slices
    assert T.int2_gemm_ws_bytes(8, 4096, 4096) == H + 2 * 8 * 4096 * 4  # 128 strips x 2 slices
    assert T.int2_gemm_ws_bytes(4, 4096, 4096) == 0  # 32 groups: unsplit below M = 5
    assert T.int2_gemm_ws_bytes(1, 2048, 8192) == 0  # 64 groups: unsplit at M = 1
    assert T.int2_gemm_ws_bytes(4, 2048, 8192) == H + 4 * 4 * 2048 * 4  # 64 groups: 4 slices at M = 4
    assert T.int2_gemm_ws_bytes(5, 14336, 4096) == 0  # 448 strips
    assert T.int2_gemm_ws_bytes(8, 4096, 512) == 0  # 4 groups: too short to slice
    assert T.int2_gemm_ws_bytes(9, 4096, 14336) == 0  # the bf16/fp16 MFMA GEMV keeps no scratch
    # the prefill GEMM's split-K partials: 4 K-slices of fp32 [M, N] where the
    # 128 x 512 tiles would leave CUs idle (8 x 8 = 64 tiles here) ...
    assert T.int2_gemm_ws_bytes(1024, 4096, 14336) == H + 4 * 1024 * 4096 * 4
    assert T.int2_gemm_ws_bytes(200, 16384, 5120) == H + 4 * 200 * 16384 * 4
    # ... and none where they fill the chip, or K is too short to slice
    assert T.int2_gemm_ws_bytes(1024, 14336, 4096) == 0
    assert T.int2_gemm_ws_bytes(256, 1024, 1024) == 0


def test_int8_ws_bytes_query():
    """The s8 x s2 GEMM's K split: the fp16 prefill GEMM's slices and partials; the decode
    GEMV's (M <= 4) strip counters in the 64 KiB workspace header and fp32 slice sums
    where K is long and the strips are few."""
    import ternocl_amd as T
    H = T.WS_HEADER_BYTES
    assert T.int2_int8_gemm_ws_bytes(1024, 4096, 14336) == H + 4 * 1024 * 4096 * 4
    assert T.int2_int8_gemm_ws_bytes(1024, 14336, 4096) == 0  # 224 wide tiles
    assert T.int2_int8_gemm_ws_bytes(4, 4096, 14336) == H + 4 * 4 * 4096 * 4  # 112 groups: 4 slices
    assert T.int2_int8_gemm_ws_bytes(1, 4096, 4096) == 0  # 32 groups
    assert T.int2_int8_gemm_ws_bytes(1, 14336, 4096) == 0  # 448 strips of 32 columns


def test_bitcos_ws_bytes_query():
    """The split BITCOS launch: a counter per 64-column strip in the workspace header
    and fp32 sums [slices][4][N]; none where one workgroup per strip fills the chip."""
    import ternocl_amd as T
    H = T.WS_HEADER_BYTES
    assert T.bitcos_gemv_ws_bytes(21504, 14) == H + 2 * 4 * 21504 * 4  # 336 strips: 2 workgroups of 7 waves each
    assert T.bitcos_gemv_ws_bytes(16384, 14) == 0  # 256 strips of 14 waves: one per CU
    assert T.bitcos_gemv_ws_bytes(21504, 12) == H + 3 * 4 * 21504 * 4  # 3 workgroups of 4 waves
    assert T.bitcos_pick_ls(1, 21504, 5376) == 12
    assert T.bitcos_pick_ls(1, 16384, 5376) == 12  # a tie at one workgroup per strip: 7 chunks per slice
    assert T.bitcos_pick_ls(1, 64, 256) == 1  # too short for 6 chunks per slice
    assert T.bitcos_gemv_ws_bytes(4096, 1) == 0
    assert T.bitcos_gemv_ws_bytes(4100, 4) == 0  # N % 16


@pytest.mark.parametrize("entry", ["ternocl_int2_moe_prefill", "ternocl_int2_moe_prefill_int8",
                                   "ternocl_int2_moe_decode"])
def test_moe_layer_host_validation(entry):
    """The MoE layer entries reject bad arguments on the host, before any device call (the
    pointers here are never dereferenced): a null weight, H % 128 != 0, a short workspace, and
    for the decode layer T * topk >= 32768."""
    import ctypes
    import ternocl_amd as T
    L = T.lib()
    fn = getattr(L, entry)
    ws_q = {"ternocl_int2_moe_prefill": lambda Tk, E, k, H, I: L.ternocl_int2_moe_prefill_ws_bytes(Tk, E, k, H, I),
            "ternocl_int2_moe_prefill_int8": lambda Tk, E, k, H, I: L.ternocl_int2_moe_prefill_int8_ws_bytes(Tk, E, k, H, I),
            "ternocl_int2_moe_decode": lambda Tk, E, k, H, I: L.ternocl_int2_moe_decode_ws_bytes(Tk, k, H, I)}[entry]
    p = ctypes.c_void_p(4096)

    def call(Tk=4, E=8, k=2, H=256, I=256, Bd=p, ws_bytes=None):
        need = ws_q(Tk, E, k, H, I)
        return fn(1, p, p, p, Tk, E, k, H, I, p, p, p, p, Bd, p, p, p, need if ws_bytes is None else ws_bytes, None)
    assert ws_q(4, 8, 2, 256, 256) > 0
    assert call(Bd=None) == 1  # TERNOCL_ERR_INVALID_ARG
    assert call(H=192) == 2  # TERNOCL_ERR_UNSUPPORTED_SHAPE
    assert call(ws_bytes=ws_q(4, 8, 2, 256, 256) - 1) == 3  # TERNOCL_ERR_WORKSPACE
    assert L.ternocl_last_error().decode()
    if entry == "ternocl_int2_moe_decode":
        assert call(Tk=4096, k=8) == 2


def test_operand_size_guards():
    """Operands the MFMA GEMMs address with 32-bit buffer offsets are rejected on
    the host at 2^31 bytes (the pointers here are never dereferenced)."""
    import ctypes
    import ternocl_amd as T
    L = T.lib()
    # prefill GEMM: K * N / 4 bytes of packed weights at 2^31
    assert _call_gemm(L, M=64, K=65536, N=131072) == 2
    p = ctypes.c_void_p(4096)
    # grouped GEMM: the gathered A rows (G / topk rows of K DT) at 2^31 bytes
    assert L.ternocl_int2_moe_gemm(1, p, p, p, 1, p, p, p, None, 8, 262144, 128, 4096, 0, 0, None) == 2
    assert L.ternocl_int2_moe_gemm(1, p, p, None, 1, p, p, p, None, 8, 1024, 1 << 21, 4096, 0, 0, None) == 2
    # MoE layers: the expert-sorted rows T * topk * I * 2 at 2^31 bytes
    for fn in (L.ternocl_int2_moe_prefill, L.ternocl_int2_moe_prefill_int8):
        assert fn(1, p, p, p, 65536, 8, 8, 2048, 2048, p, p, p, p, p, p, p, p, 1 << 40, None) == 2
    assert "2^31" in L.ternocl_last_error().decode()
    # s8 x s2 GEMM: int8 A (M * K bytes) at 2^31
    assert L.ternocl_int2_int8_gemm(0, None, p, p, p, p, p, None, None, 65536, 4096, 32768, 0, 0, None) == 2
    assert "2^31" in L.ternocl_last_error().decode()
    # M-tiled BITCOS: the re-packed int2 weights (K * N / 4 bytes of workspace) at 2^31
    assert L.ternocl_bitcos_fp16_upcvt_gemm_mt(0, p, p, p, None, 1, p, None, None, 64, 131072, 65536, 0, 0,
                                               p, 1 << 40, None) == 2
    assert "2^31" in L.ternocl_last_error().decode()
    # the decode-removed measurement kernel: B at 2^31 bytes
    assert L.ternocl_int2_gemv_stream_probe(0, p, p, p, 1, 131072, 65536, None) == 2


def test_ws_header_everywhere():
    """Every workspace size counts the 64 KiB header that holds the K splits' counters,
    so one zeroed workspace can serve any sequence of entries: the MoE layers and the
    M-tiled BITCOS re-pack place their buffers after it too."""
    import ternocl_amd as T
    L = T.lib()
    H = T.WS_HEADER_BYTES
    assert H == 64 << 10
    assert T.bitcos_gemm_mt_ws_bytes(5376, 21504) == H + 5376 // 16 * 21504 * 4
    for q in (L.ternocl_int2_moe_prefill_ws_bytes(64, 8, 2, 256, 256),
              L.ternocl_int2_moe_prefill_int8_ws_bytes(64, 8, 2, 256, 256)):
        assert q > H
    assert L.ternocl_int2_moe_decode_ws_bytes(1, 8, 256, 256) == H + 2 * 8 * 256 * 4 + 8 * 256 * 4


def test_noalloc_decode_rejects_oversized_scratch():
    """The allocation-free MoE decode entry rejects, on the host, a layer whose scratch
    exceeds its fixed 16 MiB array.  Run without a GPU on purpose: the pointers are never
    dereferenced, and a regressed check would reach the HIP runtime and fail there (a
    status other than 3), never launch a kernel."""
    import ctypes
    import ternocl_amd as T
    L = T.lib()
    p = ctypes.c_void_p(4096)
    Tk, topk, H, I = 64, 8, 4096, 8192  # 2 * 512 * 8192 * 4 bytes of gate/up rows: 32 MiB > 16 MiB
    assert L.ternocl_int2_moe_decode_ws_bytes(Tk, topk, H, I) > 16 << 20
    assert L.ternocl_int2_moe_decode_noalloc(1, p, p, p, Tk, 8, topk, H, I, p, p, p, p, p, p, p, None) == 3
    assert "16 MiB" in L.ternocl_last_error().decode()
