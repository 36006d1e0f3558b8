"""MFMA-tiled resident weight layout (apus_hip_pack_weights_dev).

The layout is restated here in numpy from its definition: for each 16-row
tile t and 128-wide K group q, the 16-byte pieces of the 64 matrix-core lanes
(lane = r + 16 g: row 16 t + r, bytes [16 g, +16) of the group's 64-byte
MXFP4 run, or of the first / second 64-byte half of the FP8 group) are stored
back to back; MXFP4 scales are [O/16][K/512][16 rows][16 bytes]. The device
packer must equal it byte for byte and unpack must invert it. GEMMs on tiled
weights must equal the same GEMMs on row-major weights bit for bit when both
run the same schedule, and match the oracle within the GEMM bar.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import acts, bf16_linear_ok, err_esc, fp4_weights, fp8_weights, max_rel

pytestmark = pytest.mark.gpu


def pack_np(fmt, w, ws, O, K):
    NQ = K // 128
    if fmt == 0:
        tw = w.reshape(O // 16, 16, NQ, 4, 16).transpose(0, 2, 3, 1, 4).reshape(w.shape)
        tws = ws.reshape(O // 16, 16, K // 512, 16).transpose(0, 2, 1, 3).reshape(ws.shape)
        return tw, tws
    tw = w.reshape(O // 16, 16, NQ, 2, 4, 16).transpose(0, 2, 3, 4, 1, 5).reshape(w.shape)
    return tw, ws


def dev_pack(hip, fmt, w, ws, O, K, unpack=False):
    L = hip.lib()
    dw, dws = hip.DevBuf.from_array(w), hip.DevBuf.from_array(ws)
    tw, tws = hip.DevBuf(w.nbytes), hip.DevBuf(ws.nbytes)
    fn = L.apus_hip_unpack_weights_dev if unpack else L.apus_hip_pack_weights_dev
    hip._check(fn(fmt, dw.ptr, dws.ptr, tw.ptr, tws.ptr, O, K), "pack")
    hip._check(L.apus_hip_synchronize(), "sync")
    out_s = tws.to_array(np.uint8, ws.shape) if fmt == 0 else ws
    return tw.to_array(np.uint8, w.shape), out_s, (tw, tws)


@pytest.mark.parametrize("fmt,O,K", [(0, 256, 2048), (0, 48, 4096), (1, 128, 4096), (1, 32, 512)])
def test_pack_matches_layout_definition(hip, rng, fmt, O, K):
    rb = K // 2 if fmt == 0 else K
    w = rng.integers(0, 256, (O, rb), dtype=np.uint8)
    ws = (rng.integers(0, 256, (O, K // 32), dtype=np.uint8) if fmt == 0
          else rng.integers(0, 256, ((O + 127) // 128, K // 128), dtype=np.uint8))
    tw, tws, _ = dev_pack(hip, fmt, w, ws, O, K)
    ew, ews = pack_np(fmt, w, ws, O, K)
    assert np.array_equal(tw, ew)
    assert np.array_equal(tws, ews)
    bw, bws, _ = dev_pack(hip, fmt, tw, tws, O, K, unpack=True)
    assert np.array_equal(bw, w) and np.array_equal(bws, ws)


def _grouped(hip, fmt, w, ws, Ms, codes, scales, O, K, flag):
    """len(Ms) entries over the same weights, consecutive activation rows."""
    L = hip.lib()
    dw, dws = hip.DevBuf.from_array(w), hip.DevBuf.from_array(ws)
    keep = [dw, dws]
    if flag:
        _, _, (tw, tws) = dev_pack(hip, fmt, w, ws, O, K)
        keep += [tw, tws]
        pw, pws = tw, (tws if fmt == 0 else dws)
    else:
        pw, pws = dw, dws
    rows = sum(Ms)
    dc, ds = hip.DevBuf.from_array(codes), hip.DevBuf.from_array(scales)
    dout = hip.DevBuf(rows * O * 4)
    ents = (hip.ApusHipGemmEnt * len(Ms))()
    m0 = 0
    for i, M in enumerate(Ms):
        ents[i] = hip.ApusHipGemmEnt(pw.ptr, pws.ptr, dout.ptr, None, None, m0, m0, M, 0)
        m0 += M
    de = hip.DevBuf(C.sizeof(ents))
    hip._check(L.apus_hip_h2d(de.ptr, C.addressof(ents), C.sizeof(ents)), "h2d")
    hip._check(L.apus_hip_gemm_grouped_dev(fmt | (hip.W_TILED if flag else 0), de.ptr, len(Ms),
                                           dc.ptr, ds.ptr, O, K, O, 0, 0), "grouped")
    hip._check(L.apus_hip_synchronize(), "sync")
    out = dout.to_array(np.float32, (rows, O)).copy()
    del keep
    return out


@pytest.mark.parametrize("fmt,O,K,Ms", [(0, 2048, 4096, [1, 5, 20, 3]),
                                        (0, 4096, 2048, [9, 1]),
                                        (1, 4096, 4096, [1, 12]),
                                        (1, 2048, 2048, [2, 70, 1, 8])])
def test_tiled_grouped_equals_rowmajor(hip, oracle, rng, fmt, O, K, Ms):
    """Enough row tiles that both layouts take the few-row and many-row
    schedules: identical bits; and the oracle's GEMM bar."""
    w, ws = (fp4_weights if fmt == 0 else fp8_weights)(rng, O, K)
    c, s = oracle.act_quant(acts(rng, sum(Ms), K, 2.0))
    row = _grouped(hip, fmt, w, ws, Ms, c, s, O, K, False)
    til = _grouped(hip, fmt, w, ws, Ms, c, s, O, K, True)
    assert np.array_equal(row.view(np.uint32), til.view(np.uint32))
    m0 = 0
    for M in Ms:
        cc, ss = c[m0:m0 + M].copy(), s[m0:m0 + M].copy()
        want = (oracle.fp4_gemm if fmt == 0 else oracle.fp8_gemm)(w, ws, cc, ss)
        truth, esc = (oracle.fp4_truth if fmt == 0 else oracle.fp8_truth)(w, ws, cc, ss)
        assert max_rel(til[m0:m0 + M], want) <= 1e-3
        assert err_esc(til[m0:m0 + M], truth, esc) <= 1e-4
        m0 += M


@pytest.mark.parametrize("fmt,M,O,K", [(0, 100, 256, 2048), (1, 70, 384, 4096),
                                       (0, 1, 2048, 4096), (1, 3, 4096, 4096),
                                       (1, 40, 256, 8192), (0, 2, 256, 1024)])
def test_tiled_dense(hip, oracle, rng, fmt, M, O, K):
    """Dense GEMM entry points on tiled weights: more than 8 rows (tile
    schedule, bitwise equal to row-major; FP8 with 9..64 rows runs the narrow
    schedule, whose four K quarters add in another order: oracle bar) and few
    rows (oracle bar)."""
    L = hip.lib()
    w, ws = (fp4_weights if fmt == 0 else fp8_weights)(rng, O, K)
    c, s = oracle.act_quant(acts(rng, M, K, 2.0))
    dc, ds = hip.DevBuf.from_array(c), hip.DevBuf.from_array(s)
    dw, dws = hip.DevBuf.from_array(w), hip.DevBuf.from_array(ws)
    _, _, (tw, tws) = dev_pack(hip, fmt, w, ws, O, K)
    fn = L.apus_hip_fp4_gemm_dev if fmt == 0 else L.apus_hip_fp8_gemm_dev
    outs = []
    for pw, pws, flag in ((dw, dws, 0), (tw, tws if fmt == 0 else dws, hip.W_TILED)):
        do = hip.DevBuf(M * O * 4)
        hip._check(fn(pw.ptr, pws.ptr, dc.ptr, ds.ptr, do.ptr, M, O, K, flag), "gemm")
        hip._check(L.apus_hip_synchronize(), "sync")
        outs.append(do.to_array(np.float32, (M, O)).copy())
    if M > 8 and not (fmt == 1 and M <= 64):
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    args = (w, ws, c, s)
    want = (oracle.fp4_gemm if fmt == 0 else oracle.fp8_gemm)(*args)
    truth, esc = (oracle.fp4_truth if fmt == 0 else oracle.fp8_truth)(*args)
    assert max_rel(outs[1], want) <= 1e-3
    assert err_esc(outs[1], truth, esc) <= 1e-4


@pytest.mark.parametrize("fmt,O,K,Ms", [(0, 2048, 4096, [1] * 12), (0, 4096, 2048, [1, 3, 8, 0, 2]),
                                        (1, 2048, 4096, [1, 7, 1]), (1, 1024, 2048, [8, 1]),
                                        (1, 1024, 4096, [1, 1, 0, 1]), (0, 1024, 2048, [1, 1])])
def test_tiled_grouped_few_rows(hip, oracle, rng, fmt, O, K, Ms):
    """Grouped launches whose entries all have at most 8 rows (max_m given)
    on tiled weights take the grouped GEMV (one row per entry or up to 8):
    every entry against the oracle's GEMM bar, entries gathering their rows
    (arows) and scattering their outputs (orows) as well as plain row
    ranges."""
    L = hip.lib()
    w, ws = (fp4_weights if fmt == 0 else fp8_weights)(rng, O, K)
    _, _, (tw, tws) = dev_pack(hip, fmt, w, ws, O, K)
    dws = hip.DevBuf.from_array(ws)
    pws = tws if fmt == 0 else dws
    rows = sum(Ms)
    c, s = oracle.act_quant(acts(rng, rows + 3, K, 2.0))
    dc, ds = hip.DevBuf.from_array(c), hip.DevBuf.from_array(s)
    dout = hip.DevBuf(rows * O * 4)                                 # plain entries
    dout2 = hip.DevBuf((rows + 2) * O * 4)                           # scattered entries
    perm = rng.permutation(rows + 3)[:rows].astype(np.int32)       # gathered rows
    operm = rng.permutation(rows + 2)[:rows].astype(np.int32)      # scattered outputs
    dperm, doperm = hip.DevBuf.from_array(perm), hip.DevBuf.from_array(operm)
    ents = (hip.ApusHipGemmEnt * len(Ms))()
    m0 = 0
    for i, M in enumerate(Ms):
        if i % 2:
            ents[i] = hip.ApusHipGemmEnt(tw.ptr, pws.ptr, dout2.ptr, dperm.ptr + 4 * m0, doperm.ptr + 4 * m0,
                                         0, 0, M, 0)
        else:
            ents[i] = hip.ApusHipGemmEnt(tw.ptr, pws.ptr, dout.ptr, None, None, m0, m0, M, 0)
        m0 += M
    de = hip.DevBuf(C.sizeof(ents))
    hip._check(L.apus_hip_h2d(de.ptr, C.addressof(ents), C.sizeof(ents)), "h2d")
    hip._check(L.apus_hip_gemm_grouped_dev(fmt | hip.W_TILED, de.ptr, len(Ms), dc.ptr, ds.ptr, O, K, O, 0,
                                           max(Ms)), "grouped")
    hip._check(L.apus_hip_synchronize(), "sync")
    out, out2 = dout.to_array(np.float32, (rows, O)), dout2.to_array(np.float32, (rows + 2, O))
    m0 = 0
    for i, M in enumerate(Ms):
        if M:
            src = perm[m0:m0 + M] if i % 2 else np.arange(m0, m0 + M)
            dst = operm[m0:m0 + M] if i % 2 else np.arange(m0, m0 + M)
            cc, ss = c[src].copy(), s[src].copy()
            want = (oracle.fp4_gemm if fmt == 0 else oracle.fp8_gemm)(w, ws, cc, ss)
            truth, esc = (oracle.fp4_truth if fmt == 0 else oracle.fp8_truth)(w, ws, cc, ss)
            got = (out2 if i % 2 else out)[dst]
            assert max_rel(got, want) <= 1e-3, i
            assert err_esc(got, truth, esc) <= 1e-4, i
        m0 += M


@pytest.mark.parametrize("fmt,M,O,K", [(1, 1, 4096, 4096), (0, 6, 2048, 4096), (1, 20, 1024, 2048),
                                       (1, 8, 1024, 8192), (0, 1, 512, 1024)])
def test_tiled_linear_dev(hip, oracle, rng, fmt, M, O, K):
    """apus_hip_linear_dev on tiled weights equals the row-major linear bit
    for bit (the same schedule for the same M), except where tiled weights
    take a schedule of their own — the split-K GEMV (FP8 and MXFP4, up to 8
    rows) and the narrow schedule (FP8, 9..64 rows): another fp32 summation
    order, so the BF16 outputs are held to the oracle's linear bar."""
    L = hip.lib()
    w, ws = (fp4_weights if fmt == 0 else fp8_weights)(rng, O, K)
    x = acts(rng, M, K)
    dx = hip.DevBuf.from_array(x)
    dw, dws = hip.DevBuf.from_array(w), hip.DevBuf.from_array(ws)
    _, _, (tw, tws) = dev_pack(hip, fmt, w, ws, O, K)
    wsp = hip.DevBuf(L.apus_hip_linear_workspace(M, K))
    outs = []
    for pw, pws, flag in ((dw, dws, 0), (tw, tws if fmt == 0 else dws, hip.W_TILED)):
        do = hip.DevBuf(M * O * 4)
        hip._check(L.apus_hip_linear_dev(fmt | flag, pw.ptr, pws.ptr, dx.ptr, do.ptr, M, K, O,
                                         wsp.ptr), "linear")
        hip._check(L.apus_hip_synchronize(), "sync")
        outs.append(do.to_array(np.float32, (M, O)).copy())
    if M <= 8 or (fmt == 1 and M <= 64):
        c, s = oracle.act_quant(x)
        unrounded = (oracle.fp4_gemm if fmt == 0 else oracle.fp8_gemm)(w, ws, c, s)
        assert bf16_linear_ok(outs[1], unrounded, 1e-4 * np.abs(unrounded).max()).all()
        return
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
