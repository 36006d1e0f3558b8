"""ctypes binding of the CPU checkers (TEST INFRASTRUCTURE ONLY).

  Oracle   : oracle/liboracle.so, the restatement of apus's quantized-matmul
             path (oracle/apus_oracle.c).
  Reference: oracle/_ref/libapus_ref.so, apus's own C kernels compiled from the
             apus sources in place (oracle/ref_shim.c, oracle/Makefile).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libapus_ref.so")

u8p = C.POINTER(C.c_uint8)
f32p = C.POINTER(C.c_float)
f64p = C.POINTER(C.c_double)
i32p = C.POINTER(C.c_int32)
i64p = C.POINTER(C.c_int64)
u64p = C.POINTER(C.c_uint64)
u32p = C.POINTER(C.c_uint32)
u8pp = C.POINTER(u8p)


def _p(a, t):
    return a.ctypes.data_as(t)


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        sz = C.c_size_t
        sig = {
            "orc_ue8m0_f32": (C.c_float, [C.c_uint8]),
            "orc_fp4_value": (C.c_float, [C.c_uint]),
            "orc_fp4_dequant_row": (None, [u8p, u8p, f32p, sz]),
            "orc_bf16_round": (C.c_float, [C.c_float]),
            "orc_e4m3_quant": (C.c_uint8, [C.c_float]),
            "orc_e4m3_dequant": (C.c_float, [C.c_uint8]),
            "orc_act_quant_row": (None, [f32p, sz, u8p, f32p]),
            "orc_act_quant_rows": (None, [f32p, sz, sz, u8p, f32p]),
            "orc_fp4_gemm": (None, [u8p, u8p, u8p, f32p, f32p, sz, sz, sz]),
            "orc_fp4_linear": (None, [u8p, u8p, f32p, f32p, sz, sz, sz]),
            "orc_fp8_gemm": (None, [u8p, u8p, u8p, f32p, f32p, sz, sz, sz]),
            "orc_fp8_linear": (None, [u8p, u8p, f32p, f32p, sz, sz, sz]),
            "orc_swiglu": (None, [f32p, f32p, f32p, sz, C.c_float]),
            "orc_moe_routed": (None, [u8pp, u8pp, u8pp, u8pp, u8pp, u8pp, C.c_int, C.c_int,
                                      C.c_float, f32p, i32p, f32p, C.c_int, C.c_int, f32p]),
            "orc_fp4_truth_f64": (None, [u8p, u8p, u8p, f32p, f64p, f64p, sz, sz, sz]),
            "orc_fp8_truth_f64": (None, [u8p, u8p, u8p, f32p, f64p, f64p, sz, sz, sz]),
            "orc_fp4_mfma_slack": (None, [u8p, u8p, u8p, f32p, f64p, sz, sz, C.c_int]),
            "orc_pin_unary": (C.c_uint64, [C.c_int, C.c_void_p, C.c_uint64, C.c_uint64,
                                           C.POINTER(C.c_uint32)]),
            "orc_hash64": (C.c_uint64, [C.c_uint64, C.c_uint64, C.c_uint64]),
            "orc_fill_bytes": (None, [C.c_uint64, C.c_uint64, C.c_uint64, u8p, sz, C.c_int]),
            "orc_wlinear": (None, [C.c_void_p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]),
            "orc_wlinear_truth_f64": (None, [C.c_void_p, f32p, f64p, f64p, C.c_int, C.c_int,
                                             C.c_int, C.c_int]),
            "orc_moe_forward": (None, [f32p, f32p, C.c_int, i64p, i64p, C.c_float, C.c_float]
                                + [u8pp] * 6 + [u8p] * 6 + [C.c_int] * 4
                                + [f32p, C.c_int, f32p, f32p, f32p, f32p, i32p, f32p]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        self.L = L

    # scalar helpers
    def ue8m0(self, b): return self.L.orc_ue8m0_f32(b)
    def fp4_value(self, n): return self.L.orc_fp4_value(n)
    def e4m3_dequant(self, c): return self.L.orc_e4m3_dequant(c)

    def fp4_dequant_row(self, packed, scales):
        K = packed.size * 2
        out = np.empty(K, np.float32)
        self.L.orc_fp4_dequant_row(_p(packed, u8p), _p(scales, u8p), _p(out, f32p), K)
        return out

    def act_quant_row(self, x):
        x = np.ascontiguousarray(x, np.float32)
        K = x.size
        codes = np.empty(K, np.uint8)
        sc = np.empty((K + 127) // 128, np.float32)
        self.L.orc_act_quant_row(_p(x, f32p), K, _p(codes, u8p), _p(sc, f32p))
        return codes, sc

    def act_quant(self, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        codes = np.empty((M, K), np.uint8)
        sc = np.empty((M, (K + 127) // 128), np.float32)
        self.L.orc_act_quant_rows(_p(x, f32p), M, K, _p(codes, u8p), _p(sc, f32p))
        return codes, sc

    def fp4_gemm(self, w, ws, acodes, asc):
        M, K = acodes.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float32)
        self.L.orc_fp4_gemm(_p(w, u8p), _p(ws, u8p), _p(acodes, u8p), _p(asc, f32p),
                            _p(out, f32p), M, O, K)
        return out

    def fp8_gemm(self, w, ws, acodes, asc):
        M, K = acodes.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float32)
        self.L.orc_fp8_gemm(_p(w, u8p), _p(ws, u8p), _p(acodes, u8p), _p(asc, f32p),
                            _p(out, f32p), M, O, K)
        return out

    def fp4_linear(self, w, ws, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float32)
        self.L.orc_fp4_linear(_p(w, u8p), _p(ws, u8p), _p(x, f32p), _p(out, f32p), M, K, O)
        return out

    def fp8_linear(self, w, ws, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float32)
        self.L.orc_fp8_linear(_p(w, u8p), _p(ws, u8p), _p(x, f32p), _p(out, f32p), M, K, O)
        return out

    def swiglu(self, g, u, limit):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        h = np.empty_like(g)
        self.L.orc_swiglu(_p(g, f32p), _p(u, f32p), _p(h, f32p), g.size, limit)
        return h

    def fp4_truth(self, w, ws, acodes, asc):
        M, K = acodes.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float64)
        esc = np.empty((M, O), np.float64)
        self.L.orc_fp4_truth_f64(_p(w, u8p), _p(ws, u8p), _p(acodes, u8p), _p(asc, f32p),
                                 _p(out, f64p), _p(esc, f64p), M, O, K)
        return out, esc

    def fp8_truth(self, w, ws, acodes, asc):
        M, K = acodes.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float64)
        esc = np.empty((M, O), np.float64)
        self.L.orc_fp8_truth_f64(_p(w, u8p), _p(ws, u8p), _p(acodes, u8p), _p(asc, f32p),
                                 _p(out, f64p), _p(esc, f64p), M, O, K)
        return out, esc

    def fp4_mfma_slack(self, w, ws, codes, scales, window):
        """The MoE checker's per-output bound on the matrix cores' block-sum
        loss (orc_fp4_mfma_slack) for one activation row."""
        w, ws = np.ascontiguousarray(w, np.uint8), np.ascontiguousarray(ws, np.uint8)
        codes = np.ascontiguousarray(np.asarray(codes).reshape(-1), np.uint8)
        scales = np.ascontiguousarray(np.asarray(scales).reshape(-1), np.float32)
        O, K = w.shape[0], codes.shape[0]
        out = np.empty(O, np.float64)
        self.L.orc_fp4_mfma_slack(_p(w, u8p), _p(ws, u8p), _p(codes, u8p), _p(scales, f32p),
                                  _p(out, f64p), O, K, window)
        return out

    def moe_routed(self, experts, x, idx, wgt, limit):
        x = np.ascontiguousarray(x, np.float32)
        idx = np.ascontiguousarray(idx, np.int32)
        wgt = np.ascontiguousarray(wgt, np.float32)
        s, dim = x.shape
        topk = idx.shape[1]
        inter = experts[0][0].shape[0]
        tabs = [(u8p * len(experts))(*[_p(e[i], u8p) for e in experts]) for i in range(6)]
        y = np.empty((s, dim), np.float32)
        self.L.orc_moe_routed(*tabs, dim, inter, limit, _p(x, f32p), _p(idx, i32p),
                              _p(wgt, f32p), s, topk, _p(y, f32p))
        return y

    def moe_forward(self, cfg, experts, shared, x):
        """orc_moe_forward: (out, routed, shared, sp, idx, wgt)."""
        keep, tabs, gw, gb, t2e, ids, sh, x, ptr, i64 = _moe_args(cfg, experts, shared, x)
        s, dim = x.shape
        E, topk = cfg["E"], cfg["topk"]
        res = [np.empty((s, dim), np.float32) for _ in range(3)]
        sp = np.empty((s, E), np.float32)
        idx = np.empty((s, topk), np.int32)
        wgt = np.empty((s, topk), np.float32)
        self.L.orc_moe_forward(_p(gw, f32p), ptr(gb, f32p), int(cfg["hash"]), ptr(t2e, i64),
                               ptr(ids, i64), C.c_float(cfg["route_scale"]),
                               C.c_float(cfg["limit"]), *tabs,
                               *[_p(a, u8p) for a in sh], E, topk, dim, cfg["inter"],
                               _p(x, f32p), s, *[_p(r, f32p) for r in res], _p(sp, f32p),
                               _p(idx, i32p), _p(wgt, f32p))
        return (*res, sp, idx, wgt)

    def wlinear(self, w, x, flags):
        """orc_wlinear: w [O, K] float32, or uint16 BF16 bits (flag 4)."""
        w = np.ascontiguousarray(w)
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        O = w.shape[0]
        assert (w.dtype == np.uint16) == bool(flags & 4)
        out = np.empty((M, O), np.float32)
        self.L.orc_wlinear(w.ctypes.data, _p(x, f32p), _p(out, f32p), M, K, O, flags)
        return out

    def wlinear_truth(self, w, x, flags):
        w = np.ascontiguousarray(w)
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        O = w.shape[0]
        t, e = np.empty((M, O), np.float64), np.empty((M, O), np.float64)
        self.L.orc_wlinear_truth_f64(w.ctypes.data, _p(x, f32p), _p(t, f64p), _p(e, f64p), M, K, O,
                                     flags)
        return t, e

    def fill_bytes(self, seed, stream, n, kind, first=0):
        out = np.empty(n, np.uint8)
        self.L.orc_fill_bytes(seed, stream, first, _p(out, u8p), n, kind)
        return out

    def pin_unary(self, which, fnptr, lo, hi):
        bad = C.c_uint32()
        n = self.L.orc_pin_unary(which, fnptr, lo, hi, C.byref(bad))
        return n, bad.value


ST_BF16, ST_F32 = 4, 6   # c/st.h:40-44 ApusStDtype


class StTensor(C.Structure):
    """c/st.h:46-53 ApusStTensor (a tensor view; the head GEMV hook takes one)."""
    _fields_ = [("name", C.c_char * 160), ("dtype", C.c_int), ("ndim", C.c_int),
                ("shape", C.c_int64 * 8), ("data", C.c_void_p), ("nbytes", C.c_size_t)]


class _WeightView(C.Structure):
    """c/st.h:88-89: {codes|packed, scales, O, K} — same layout for fp8 and fp4."""
    _fields_ = [("w", C.c_void_p), ("s", C.c_void_p), ("O", C.c_int64), ("K", C.c_int64)]


def _moe_args(cfg, experts, shared, x):
    """Argument tuple shared by orc_moe_forward and ref_moe_forward.
    cfg: dict E, topk, dim, inter, route_scale, limit, hash, gate_w [E, dim],
    gate_bias [E] or None, tid2eid [n, topk] int64 or None, ids [s] int64 or
    None; experts: E tuples (w1, w1s, w2, w2s, w3, w3s); shared: FP8 (sw1,
    sw1s, sw2, sw2s, sw3, sw3s)."""
    keep = []

    def arr(a, dt):
        a = np.ascontiguousarray(a, dt)
        keep.append(a)
        return a
    gw = arr(cfg["gate_w"], np.float32)
    gb = arr(cfg["gate_bias"], np.float32) if cfg.get("gate_bias") is not None else None
    t2e = arr(cfg["tid2eid"], np.int64) if cfg.get("tid2eid") is not None else None
    ids = arr(cfg["ids"], np.int64) if cfg.get("ids") is not None else None
    tabs = [(u8p * len(experts))(*[_p(e[i], u8p) for e in experts]) for i in range(6)]
    sh = [arr(a, np.uint8) for a in shared]
    x = arr(x, np.float32)
    i64 = C.POINTER(C.c_int64)
    ptr = lambda a, t: _p(a, t) if a is not None else None  # noqa: E731
    return keep, tabs, gw, gb, t2e, ids, sh, x, ptr, i64


class Reference:
    """apus's own CPU kernels (compiled from the apus sources)."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where the apus "
                                    "sources are present")
        L = C.CDLL(path)
        sz = C.c_size_t
        sig = {
            "apus_ue8m0_f32": (C.c_float, [C.c_uint8]),
            "apus_e4m3_quant_f32": (C.c_uint8, [C.c_float]),
            "apus_e4m3_dequant_f32": (C.c_float, [C.c_uint8]),
            "apus_bf16_round": (C.c_float, [C.c_float]),
            "apus_fp4_act_quant_scalar": (None, [f32p, sz, u8p, f32p]),
            "apus_fp4_dequant_row_scalar": (None, [u8p, u8p, f32p, sz]),
            "apus_fp4_gemm_scalar": (None, [u8p, u8p, u8p, f32p, f32p, f32p, sz, sz, sz]),
            "apus_fp4_gemm_mt": (None, [u8p, u8p, u8p, f32p, f32p, f32p, sz, sz, sz]),
            "apus_fp8_gemm_scalar": (None, [u8p, u8p, u8p, f32p, f32p, f32p, sz, sz, sz]),
            "apus_fp8_gemm_mt": (None, [u8p, u8p, u8p, f32p, f32p, f32p, sz, sz, sz]),
            "apus_fp4_linear": (None, [C.c_void_p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
            "apus_fp8_linear": (None, [C.c_void_p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
            "ref_swiglu": (None, [f32p, f32p, f32p, sz, C.c_float]),
            "ref_act_quant_rows": (None, [f32p, C.c_int, C.c_int, f32p, u8p, f32p]),
            "ref_x86_avx2_hits": (C.c_ulong, []),
            "ref_pool_threads": (C.c_int, []),
            "ref_moe_routed": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float,
                                         f32p, u8pp, u8pp, u8pp, u8pp, u8pp, u8pp, f32p, i32p,
                                         C.c_int, f32p, f32p, f32p]),
            "ref_moe_forward": (None, [C.c_int] * 4 + [C.c_float, C.c_float, C.c_int, f32p, f32p,
                                                        i64p, i64p] + [u8pp] * 6 + [u8p] * 6
                                + [f32p, C.c_int, f32p, f32p, f32p, f32p, i32p, f32p]),
            "ref_decode_layer": (None, [C.c_int, C.c_int, C.c_int, C.c_float] + [u8pp] * 6
                                 + [f32p, u8p, u8p, C.c_int, f32p, f32p, f32p]),
            "apus_f32_linear": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
            "apus_bf16_linear": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
            "apus_head_gemv": (None, [C.c_void_p, f32p, f32p, C.c_int64, C.c_int64]),
            "ref_store_index": (C.c_int, [C.c_char_p, C.c_int, C.c_int, C.c_int, i32p, u64p, u64p,
                                          u32p, i64p, i64p, C.c_char_p, C.c_int,
                                          C.POINTER(C.c_int), u8p, C.c_char_p, C.c_size_t]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        self.L = L

    def act_quant(self, x):
        """c/attn.h:393-403: BF16 round then apus_fp4_act_quant_scalar per row."""
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        xb = np.empty_like(x)
        codes = np.empty((M, K), np.uint8)
        sc = np.empty((M, (K + 127) // 128), np.float32)
        self.L.ref_act_quant_rows(_p(x, f32p), M, K, _p(xb, f32p), _p(codes, u8p), _p(sc, f32p))
        return codes, sc

    def _gemm(self, fn, w, ws, acodes, asc):
        M, K = acodes.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float32)
        scratch = np.empty(M * K * 2 + 64, np.float32)
        fn(_p(w, u8p), _p(ws, u8p), _p(acodes, u8p), _p(asc, f32p), _p(scratch, f32p),
           _p(out, f32p), M, O, K)
        return out

    def fp4_gemm_scalar(self, *a): return self._gemm(self.L.apus_fp4_gemm_scalar, *a)
    def fp4_gemm_mt(self, *a): return self._gemm(self.L.apus_fp4_gemm_mt, *a)
    def fp8_gemm_scalar(self, *a): return self._gemm(self.L.apus_fp8_gemm_scalar, *a)
    def fp8_gemm_mt(self, *a): return self._gemm(self.L.apus_fp8_gemm_mt, *a)

    def _linear(self, fn, w, ws, x, fp4):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        O = w.shape[0]
        out = np.empty((M, O), np.float32)
        view = _WeightView(w.ctypes.data, ws.ctypes.data, O, K)   # ApusFp4W / ApusFp8W
        fn(C.addressof(view), _p(x, f32p), _p(out, f32p), M, K, O)
        return out

    def fp4_linear(self, w, ws, x): return self._linear(self.L.apus_fp4_linear, w, ws, x, True)
    def fp8_linear(self, w, ws, x): return self._linear(self.L.apus_fp8_linear, w, ws, x, False)

    def swiglu(self, g, u, limit):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        h = np.empty_like(g)
        self.L.ref_swiglu(_p(g, f32p), _p(u, f32p), _p(h, f32p), g.size, limit)
        return h

    def f32_linear(self, w, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        out = np.empty((M, w.shape[0]), np.float32)
        self.L.apus_f32_linear(_p(np.ascontiguousarray(w, np.float32), f32p), _p(x, f32p),
                               _p(out, f32p), M, K, w.shape[0])
        return out

    def bf16_linear(self, w, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        out = np.empty((M, w.shape[0]), np.float32)
        self.L.apus_bf16_linear(_p(np.ascontiguousarray(w, np.float32), f32p), _p(x, f32p),
                                _p(out, f32p), M, K, w.shape[0])
        return out

    def head_gemv(self, w, x):
        """apus_head_gemv over an F32 (float32 w) or BF16 (uint16 w) view."""
        w = np.ascontiguousarray(w)
        x = np.ascontiguousarray(x, np.float32).ravel()
        O, K = w.shape
        t = StTensor()
        t.name = b"head"
        t.dtype = ST_BF16 if w.dtype == np.uint16 else ST_F32
        t.ndim = 2
        t.shape[0], t.shape[1] = O, K
        t.data = w.ctypes.data
        t.nbytes = w.nbytes
        out = np.empty(O, np.float32)
        self.L.apus_head_gemv(C.byref(t), _p(x, f32p), _p(out, f32p), O, K)
        return out

    def store_index(self, path, n_layers, n_mtp, E, with_slabs=False):
        """The reference expert store's slab records (apus_store_open):
        ([(shard_name, off, len, rel[6], O[3], K[3])] layer-major, slabs or
        None), or raises ValueError with the reference's message."""
        n = n_layers * E
        shard = np.zeros(n, np.int32)
        off, ln = np.zeros(n, np.uint64), np.zeros(n, np.uint64)
        rel = np.zeros((n, 6), np.uint32)
        O, K = np.zeros((n, 3), np.int64), np.zeros((n, 3), np.int64)
        cap = 256
        names = C.create_string_buffer(cap * 64)
        nn = C.c_int()
        err = C.create_string_buffer(512)
        # slabs are sized after a first pass that learns the slab length
        rc = self.L.ref_store_index(path.encode(), n_layers, n_mtp, E, _p(shard, i32p),
                                    _p(off, u64p), _p(ln, u64p), _p(rel, u32p), _p(O, i64p),
                                    _p(K, i64p), names, cap, C.byref(nn), None, err, 512)
        if rc:
            raise ValueError(err.value.decode())
        slabs = None
        if with_slabs:
            slabs = np.zeros((n, int(ln.max())), np.uint8)
            rc = self.L.ref_store_index(path.encode(), n_layers, n_mtp, E, _p(shard, i32p),
                                        _p(off, u64p), _p(ln, u64p), _p(rel, u32p), _p(O, i64p),
                                        _p(K, i64p), names, cap, C.byref(nn), _p(slabs, u8p),
                                        err, 512)
            if rc:
                raise ValueError(err.value.decode())
        nm = [names.raw[k * cap:(k + 1) * cap].split(b"\0")[0].decode() for k in range(nn.value)]
        recs = [(nm[shard[i]], int(off[i]), int(ln[i]), rel[i].tolist(), O[i].tolist(), K[i].tolist())
                for i in range(n)]
        return recs, slabs

    def moe_forward(self, cfg, experts, shared, x):
        """The real apus_moe_forward: (out, routed, shared, sp, idx, wgt)."""
        keep, tabs, gw, gb, t2e, ids, sh, x, ptr, i64 = _moe_args(cfg, experts, shared, x)
        s, dim = x.shape
        E, topk = cfg["E"], cfg["topk"]
        res = [np.empty((s, dim), np.float32) for _ in range(3)]
        sp = np.empty((s, E), np.float32)
        idx = np.empty((s, topk), np.int32)
        wgt = np.empty((s, topk), np.float32)
        self.L.ref_moe_forward(E, topk, dim, cfg["inter"], C.c_float(cfg["route_scale"]),
                               C.c_float(cfg["limit"]), int(cfg["hash"]), _p(gw, f32p),
                               ptr(gb, f32p), ptr(t2e, i64), ptr(ids, i64), *tabs,
                               *[_p(a, u8p) for a in sh], _p(x, f32p), s,
                               *[_p(r, f32p) for r in res], _p(sp, f32p), _p(idx, i32p),
                               _p(wgt, f32p))
        return (*res, sp, idx, wgt)

    def moe_routed(self, experts, gate_w, x, idx, route_scale, limit):
        """Real apus_moe_forward with idx forced through hash routing; returns
        (router_w, routed_y)."""
        x = np.ascontiguousarray(x, np.float32)
        idx = np.ascontiguousarray(idx, np.int32)
        gate_w = np.ascontiguousarray(gate_w, np.float32)
        s, dim = x.shape
        topk = idx.shape[1]
        E = len(experts)
        inter = experts[0][0].shape[0]
        tabs = [(u8p * E)(*[_p(e[i], u8p) for e in experts]) for i in range(6)]
        rw = np.empty((s, topk), np.float32)
        y = np.empty((s, dim), np.float32)
        out = np.empty((s, dim), np.float32)
        rc = self.L.ref_moe_routed(E, topk, dim, inter, route_scale, limit, _p(gate_w, f32p),
                                   *tabs, _p(x, f32p), _p(idx, i32p), s, _p(rw, f32p),
                                   _p(y, f32p), _p(out, f32p))
        if rc != 0:
            raise RuntimeError("reference routing did not follow the forced expert ids")
        return rw, y


def ref_decode_layer(R, experts, wgt, pw, pws, x, limit):
    """One token through one config-4 layer on apus's own CPU kernels
    (ref_decode_layer): experts = topk tuples (w1, w1s, w2, w2s, w3, w3s),
    wgt [topk], FP8 projection pw [O8, dim] / pws; returns (y, proj)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    dim = x.shape[0]
    topk = len(experts)
    inter = experts[0][0].shape[0]
    tabs = [(u8p * topk)(*[_p(e[i], u8p) for e in experts]) for i in range(6)]
    wgt = np.ascontiguousarray(wgt, np.float32)
    y = np.empty(dim, np.float32)
    proj = np.empty(pw.shape[0], np.float32)
    R.L.ref_decode_layer(topk, dim, inter, limit, *tabs, _p(wgt, f32p), _p(pw, u8p), _p(pws, u8p),
                         pw.shape[0], _p(x, f32p), _p(y, f32p), _p(proj, f32p))
    return y, proj


def bf16_round_np(x):
    """Vectorised BF16 RNE (same rule as orc_bf16_round), for input prep."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(nan, x.view(np.uint32), r)
    return r.view(np.float32).reshape(x.shape)


def have_ref():
    return os.path.exists(REF_SO)
