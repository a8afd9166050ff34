"""Compact-i4 embedding rows on the GPU (tqhip_dequant_i4_rows_dev) against the
oracle's dequant_i4_row, which tests/test_oracle.py pins to the reference's
golden table and known answers (tests/test_quant_ops.cpp:62-112). One fp32
subtraction and one product per element, as the reference: bit-exact."""
import numpy as np
import pytest

from conftest import golden

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def gather(gpu, table, rows, dim, G):
    dt = gpu.DeviceBuffer.from_array(np.ascontiguousarray(table, np.uint8))
    r = np.asarray(rows, np.int32)
    dr = gpu.DeviceBuffer.from_array(r)
    dout = gpu.DeviceBuffer(4 * dim * len(r))
    gpu.dequant_i4_rows_dev(dt, dr, len(r), dim, G, dout)
    gpu.synchronize()
    return dout.download(np.float32, dim * len(r)).reshape(len(r), dim)


def test_golden_table_rows(gpu):
    f = golden("dequant_i4_row")
    nrows, dim, G = (int(v) for v in f["dims"])
    got = gather(gpu, f["table"], list(range(nrows)) + [3, 0], dim, G)
    want = np.concatenate([f["table_rows"], f["table_rows"][[3, 0]]])
    assert np.array_equal(bits(got), bits(want))
    kat = gather(gpu, f["kat_embed"], [0], 8, 4)[0]  # tests/test_quant_ops.cpp:87
    assert np.array_equal(kat, np.array([-4, 0, 3.5, -2.5, 0, 0, 0, 0], np.float32))


@pytest.mark.parametrize("vocab,dim,G", [(1000, 896, 64), (300, 2560, 64), (77, 200, 64), (50, 1000, 128),
                                         (9, 70, 6), (40, 100, 32)])
def test_random_tables_match_oracle(gpu, orc, vocab, dim, G):
    table = gpu.synth_i4(vocab, dim, G, seed=vocab + dim)
    rng = np.random.default_rng(G)
    rows = rng.integers(0, vocab, 33)
    got = gather(gpu, table, rows, dim, G)
    for t, r in enumerate(rows):
        assert np.array_equal(bits(got[t]), bits(orc.dequant_i4_row(table, int(r), dim, G))), f"row {r}"
