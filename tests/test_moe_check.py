"""The stage-wise MoE checker (moe_check.py) on the CPU: it accepts the
oracle's own dispatch intermediates, and rejects plausible mistakes (a scale
byte off by one, two h codes swapped, one code moved by a step, a wrong
expert's w2, a y one fp32 ulp off where every eo is pinned, a y perturbed
by 1e-3 relative at its largest element, a dropped routing weight)."""
import numpy as np
import pytest

from helpers import acts, bf16, moe_experts, topk_routing
from moe_check import check_token

DIM, INTER, E, TOPK = 512, 256, 8, 4


def oracle_token(oracle, experts, x_row, idx_row, wgt_row, limit):
    """The dispatch of one token through the oracle's own steps: h codes and
    E8M0 bytes per pair and y, as the GPU would hand them over."""
    xc, xs = oracle.act_quant(bf16(x_row[None, :]))
    hc, he, eo = [], [], []
    for e in idx_row:
        w1, w1s, w2, w2s, w3, w3s = experts[int(e)]
        g = bf16(oracle.fp4_gemm(w1, w1s, xc, xs))
        u = bf16(oracle.fp4_gemm(w3, w3s, xc, xs))
        h = oracle.swiglu(g, u, limit)
        c, s = oracle.act_quant(h)
        hc.append(c[0])
        he.append((s[0].view(np.uint32) >> 23).astype(np.uint8))
        eo.append(bf16(oracle.fp4_gemm(w2, w2s, c, s))[0])
    y = np.zeros(DIM, np.float32)
    for j in range(len(idx_row)):
        y = (y + (np.float32(wgt_row[j]) * eo[j]).astype(np.float32)).astype(np.float32)
    return np.stack(hc), np.stack(he), y


@pytest.fixture(scope="module")
def case(oracle):
    rng = np.random.default_rng(5)
    experts = moe_experts(rng, E, DIM, INTER)
    x = acts(rng, 1, DIM)
    idx, wgt = topk_routing(rng, 1, E, TOPK)
    hc, he, y = oracle_token(oracle, experts, x[0], idx[0], wgt[0], 10.0)
    return experts, x[0], idx[0], wgt[0], hc, he, y


def run(oracle, case, hc=None, he=None, y=None, idx=None, wgt=None):
    experts, x, idx0, wgt0, hc0, he0, y0 = case
    return check_token(oracle, lambda e: experts[e], x, idx0 if idx is None else idx,
                       wgt0 if wgt is None else wgt, 10.0,
                       hc0 if hc is None else hc, he0 if he is None else he,
                       y0 if y is None else y)


def test_accepts_oracle(oracle, case):
    r = run(oracle, case)
    assert r["h_pinned"] > 0.95 and r["y_pinned"] > 0.1, r


def test_rejects_scale_byte(oracle, case):
    he = case[5].copy()
    he[1, 0] += 1
    with pytest.raises(AssertionError):
        run(oracle, case, he=he)


def test_rejects_swapped_codes(oracle, case):
    hc = case[4].copy()
    k = int(np.argmax(np.abs(hc[0].astype(np.int16) - hc[0, ::-1].astype(np.int16))))
    hc[0, [k, -1 - k]] = hc[0, [-1 - k, k]]
    with pytest.raises(AssertionError):
        run(oracle, case, hc=hc)


def test_rejects_one_code_step(oracle, case):
    hc = case[4].copy()
    k = int(np.nonzero((hc[2] & 0x7F) > 8)[0][0])
    hc[2, k] = hc[2, k] + 1
    with pytest.raises(AssertionError):
        run(oracle, case, hc=hc)


def test_rejects_wrong_expert(oracle, case):
    idx = case[2].copy()
    idx[3] = (idx[3] + 1) % E if (idx[3] + 1) % E not in idx else (idx[3] + 2) % E
    with pytest.raises(AssertionError):
        run(oracle, case, idx=idx)


def test_rejects_one_ulp_where_pinned(oracle, case):
    pin = run(oracle, case)["y_pinned_mask"]
    y = case[6].copy()
    k = int(np.argmax(np.where(pin, np.abs(y), -1.0)))
    assert pin[k]
    y[k] = np.nextafter(y[k], np.float32(np.inf))
    with pytest.raises(AssertionError):
        run(oracle, case, y=y)


def test_rejects_small_y_error(oracle, case):
    y = case[6].copy()
    k = int(np.argmax(np.abs(y)))
    y[k] *= np.float32(1 + 1e-3)
    with pytest.raises(AssertionError):
        run(oracle, case, y=y)


def test_rejects_dropped_weight(oracle, case):
    wgt = case[3].copy()
    wgt[-1] = 0.0
    with pytest.raises(AssertionError):
        run(oracle, case, wgt=wgt)
