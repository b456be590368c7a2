"""The C ABI's host packers (ternocl_int2_pack / _unpack, ternocl_bitcos_pack /
_unpack / _pack_words, ternocl_bitcos_slice_ranks_host), on the CPU.

Bars: bit-exact against the numpy formats (ternocl_amd/formats.py, an
independent restatement), against the oracle's packer, and against buffers the
reference's own generator built (common/bitcos.hpp:31-78 bitcos_random,
compiled into oracle/_ref): decoding such a buffer and packing the codes again
must give it back word for word.  The packers take dense ternary weights
int8 [K, N]; anything else is rejected with a status.
"""
from __future__ import annotations

import numpy as np
import pytest

import ternocl_amd as T
from ternocl_amd import formats, synth


def _ternary(g, K, N, z):
    """iid ternary values, P(0) = z, P(+1) = P(-1) = (1 - z) / 2."""
    u = g.random((K, N))
    return np.where(u < z, 0, np.where(u < z + (1 - z) / 2, 1, -1)).astype(np.int8)


@pytest.mark.parametrize("K,N", [(16, 1), (128, 48), (4096, 272), (256, 16), (1024, 1000)])
def test_int2_pack_matches_formats_and_round_trips(K, N):
    g = synth.rng(K + N)
    W = _ternary(g, K, N, 0.5)
    B = T.int2_pack(W)
    assert np.array_equal(B, formats.pack_int2(W))
    assert np.array_equal(T.int2_unpack(B, K), W)
    # unpack reads every code, code 2 as -2 (formats.unpack_int2's two's complement)
    R = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)
    assert np.array_equal(T.int2_unpack(R, K), formats.unpack_int2(R, K))


def test_int2_pack_codes_of_each_value():
    W = np.zeros((16, 3), np.int8)
    W[:, 1] = 1
    W[:, 2] = -1
    W[5, 0] = -1
    B = T.int2_pack(W)
    assert B[0, 0] == 3 << 10
    assert B[0, 1] == 0x55555555
    assert B[0, 2] == 0xFFFFFFFF


def test_int2_pack_rejects_bad_input():
    with pytest.raises(T.TernoclError):
        T.int2_pack(np.full((16, 4), 2, np.int8))  # not ternary
    with pytest.raises(T.TernoclError):
        T.int2_pack(np.zeros((24, 4), np.int8))  # K % 16


@pytest.mark.parametrize("z", [0.0, 0.3, 0.5, 0.7, 1.0])
@pytest.mark.parametrize("K,N", [(32, 1), (1024, 48), (5376, 64)])
def test_bitcos_pack_matches_formats(z, K, N):
    g = synth.rng(int(z * 10) + K + N)
    W = _ternary(g, K, N, z)
    if N > 2:  # a column of zeros, a full column and nnz = 32 exactly
        W[:, 0] = 0
        W[:, 1] = np.where(g.random(K) < 0.5, 1, -1)
        W[:, 2] = 0
        W[:32, 2] = -1
    buf = T.bitcos_pack(W)
    assert buf.size == T.lib().ternocl_bitcos_pack_words(W.ctypes.data, K, N)
    assert np.array_equal(buf, formats.bitcos_pack(W))
    assert np.array_equal(T.bitcos_unpack(buf, K, N), W)
    for ls in (1, 2, 3, 7, 14):
        assert np.array_equal(T.bitcos_slice_ranks_host(buf, K, N, ls), formats.bitcos_slice_ranks(buf, K, N, ls))


def test_bitcos_pack_matches_the_oracle(orc):
    g = synth.rng(3)
    W = _ternary(g, 512, 80, 0.4)
    assert np.array_equal(T.bitcos_pack(W), orc.bitcos_pack(W))


@pytest.mark.skipif(not __import__("oracle.binding", fromlist=["x"]).ref_available(),
                    reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("z", [0.3, 0.5, 0.7])
def test_bitcos_pack_reproduces_the_reference_generator(orc, z):
    """bitcos_random's buffer -> unpack -> pack gives the same words; the
    unpack equals the reference's bitcos_decode_col and the slice ranks its
    bitcos_slice_ranks."""
    K, N = 1024, 96
    buf = orc.ref_bitcos_random(K, N, z, 4321)
    W = T.bitcos_unpack(buf, K, N)
    assert np.array_equal(W, orc.ref_bitcos_decode(buf, K, N))
    assert np.array_equal(T.bitcos_pack(W), buf)
    for ls in (1, 2, 4, 8):
        assert np.array_equal(T.bitcos_slice_ranks_host(buf, K, N, ls), orc.ref_bitcos_slice_ranks(buf, K, N, ls))


def test_bitcos_pack_rejects_bad_input():
    L = T.lib()
    W = np.zeros((64, 16), np.int8)
    assert L.ternocl_bitcos_pack_words(np.full((64, 16), 3, np.int8).ctypes.data, 64, 16) == 0
    assert L.ternocl_bitcos_pack_words(W.ctypes.data, 48, 16) == 0  # K % 32
    n = L.ternocl_bitcos_pack_words(W.ctypes.data, 64, 16)
    buf = np.zeros(n - 1, np.uint32)
    assert L.ternocl_bitcos_pack(W.ctypes.data, 64, 16, buf.ctypes.data, n - 1) != 0  # short buffer
    bad = np.zeros(64 // 32 * 16 + 16, np.uint32)  # no room for the pad words
    with pytest.raises(T.TernoclError):
        T.bitcos_unpack(bad, 64, 16)
