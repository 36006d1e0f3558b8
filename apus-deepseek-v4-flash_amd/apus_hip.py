"""ctypes binding of libapus_hip.so (include/apus_hip.h) for tests and benchmarks.

The product is the C ABI; this module only marshals numpy arrays into it.
Names follow the reference entry points they replace:
  act_quant   -> c/attn.h:393-403 + c/fp4.h:293-321 (apus_act_quant_rows)
  fp4_gemm    -> c/fp4.h:815 apus_fp4_gemm_mt
  fp8_gemm    -> c/fp8.h:557 apus_fp8_gemm_mt
  fp4_linear  -> c/attn.h:432 apus_fp4_linear
  fp8_linear  -> c/attn.h:408 apus_fp8_linear
  fp4_gemm_grouped -> c/fp4.h:936 apus_fp4_gemm_mt_grouped
  moe_routed  -> routed dispatch of c/moe.h:433-563 (apus_moe_forward)
Every call raises ApusHipError when the backend reports "unsupported" or
fails, and loading raises when the shared library is missing: there is no
CPU fallback in this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libapus_hip.so")
W_TILED = 0x100        # APUS_HIP_W_TILED: weights in the MFMA-tiled layout

u8p = C.POINTER(C.c_uint8)
f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)
vp = C.c_void_p


class ApusHipError(RuntimeError):
    pass


class ApusFp8W(C.Structure):
    _fields_ = [("codes", u8p), ("scales", u8p), ("O", C.c_int64), ("K", C.c_int64)]


class ApusFp4W(C.Structure):
    _fields_ = [("packed", u8p), ("scales", u8p), ("O", C.c_int64), ("K", C.c_int64)]


class ApusFp4GemmEnt(C.Structure):
    _fields_ = [("w", u8p), ("ws", u8p), ("out", f32p), ("m0", C.c_size_t), ("M", C.c_size_t)]


RESOLVE_FN = C.CFUNCTYPE(C.c_int, vp, C.c_int, C.c_int, C.POINTER(ApusFp4W),
                         C.POINTER(ApusFp4W), C.POINTER(ApusFp4W))
HINT_FN = C.CFUNCTYPE(None, vp, C.c_int, C.c_int)
END_FN = C.CFUNCTYPE(None, vp, C.c_int)


class ApusMoeW(C.Structure):
    _fields_ = [("E", C.c_int), ("topk", C.c_int), ("inter", C.c_int), ("dim", C.c_int),
                ("hash", C.c_int), ("route_scale", C.c_float), ("limit", C.c_float),
                ("gate_w", f32p), ("gate_bias", f32p), ("tid2eid", C.POINTER(C.c_int64)),
                ("w1", C.POINTER(ApusFp4W)), ("w2", C.POINTER(ApusFp4W)),
                ("w3", C.POINTER(ApusFp4W)),
                ("sw1", ApusFp8W), ("sw2", ApusFp8W), ("sw3", ApusFp8W),
                ("hook_ctx", vp), ("hook_resolve", RESOLVE_FN), ("hook_hint", HINT_FN),
                ("hook_layer_end", END_FN), ("hook_hint_ctx", vp),
                ("hook_layer_end_ctx", vp), ("layer_id", C.c_int)]


class ApusHipGemmEnt(C.Structure):
    _fields_ = [("w", vp), ("ws", vp), ("out", vp), ("arows", vp), ("orows", vp),
                ("a0", C.c_int32), ("o0", C.c_int32), ("M", C.c_int32), ("reserved", C.c_int32)]


HOOK_FIELDS = ("fp8_linear", "f32_linear", "head_gemv", "fp4_linear", "fp4_gemm_grouped",
               "moe_routed")


class ApusHipHooks(C.Structure):
    _fields_ = [(n, vp) for n in HOOK_FIELDS]


class ApusHipMoeLayer(C.Structure):
    """Router and shared-expert weights of one MoE layer (device pointers)."""
    _fields_ = [("gate_w", vp), ("gate_bias", vp), ("tid2eid", vp), ("hash", C.c_int),
                ("route_scale", C.c_float), ("limit", C.c_float),
                ("sw1", vp), ("sw1s", vp), ("sw2", vp), ("sw2s", vp), ("sw3", vp), ("sw3s", vp),
                ("shared_tiled", C.c_int)]


class ApusHipMoeInterm(C.Structure):
    """Optional device outputs of apus_hip_moe_forward_dev (c/moe.h:64-71)."""
    _fields_ = [("router_scores", vp), ("router_idx", vp), ("router_w", vp),
                ("moe_routed", vp), ("moe_shared", vp)]

class ApusHipSlabRec(C.Structure):
    """One routed expert's slab in an apus container (include/apus_hip.h)."""
    _fields_ = [("shard", C.c_int32), ("pad", C.c_int32), ("off", C.c_uint64), ("len", C.c_uint64),
                ("rel", C.c_uint32 * 6), ("O", C.c_int64 * 3), ("K", C.c_int64 * 3)]

# entry point -> (restype, argtypes); exactly the declarations of include/apus_hip.h
SIGNATURES = {
    "apus_hip_enable": (C.c_int, [C.c_char_p, C.c_size_t]),
    "apus_hip_disable": (None, []),
    "apus_hip_is_enabled": (C.c_int, []),
    "apus_hip_hooks": (C.POINTER(ApusHipHooks), []),
    "apus_hip_bytes_uploaded": (C.c_uint64, []),
    "apus_hip_bytes_resident": (C.c_uint64, []),
    "apus_hip_dispatches": (C.c_uint64, []),
    "apus_hip_fp8_linear": (C.c_int, [C.POINTER(ApusFp8W), f32p, f32p, C.c_int, C.c_int, C.c_int]),
    "apus_hip_fp4_linear": (C.c_int, [C.POINTER(ApusFp4W), f32p, f32p, C.c_int, C.c_int, C.c_int]),
    "apus_hip_fp4_gemm_grouped": (C.c_int, [C.POINTER(ApusFp4GemmEnt), C.c_size_t, u8p, f32p,
                                            C.c_size_t, C.c_size_t]),
    "apus_hip_moe_routed": (C.c_int, [C.POINTER(ApusMoeW), f32p, i32p, f32p, C.c_int, f32p]),
    "apus_hip_f32_linear": (C.c_int, [vp, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]),
    "apus_hip_head_gemv": (C.c_int, [vp, f32p, f32p, C.c_int64, C.c_int64]),
    "apus_hip_wlinear_dev": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int]),
    "apus_hip_act_quant": (C.c_int, [f32p, C.c_int, C.c_int, u8p, f32p]),
    "apus_hip_fp4_gemm": (C.c_int, [u8p, u8p, u8p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
    "apus_hip_fp8_gemm": (C.c_int, [u8p, u8p, u8p, f32p, f32p, C.c_int, C.c_int, C.c_int]),
    "apus_hip_swiglu_dev": (C.c_int, [vp, vp, C.c_size_t, C.c_float, vp]),
    "apus_hip_act_quant_dev": (C.c_int, [vp, C.c_int, C.c_int, vp, vp]),
    "apus_hip_fp4_gemm_dev": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int]),
    "apus_hip_fp8_gemm_dev": (C.c_int, [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_int]),
    "apus_hip_gemm_grouped_dev": (C.c_int, [C.c_int, vp, C.c_int, vp, vp, C.c_int, C.c_int,
                                            C.c_int, C.c_int, C.c_int]),
    "apus_hip_store_tiled": (C.c_int, [vp]),
    "apus_hip_linear_dev": (C.c_int, [C.c_int, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp]),
    "apus_hip_pack_weights_dev": (C.c_int, [C.c_int, vp, vp, vp, vp, C.c_int, C.c_int]),
    "apus_hip_unpack_weights_dev": (C.c_int, [C.c_int, vp, vp, vp, vp, C.c_int, C.c_int]),
    "apus_hip_linear_workspace": (C.c_size_t, [C.c_int, C.c_int]),
    "apus_hip_fp4_linear_dev": (C.c_int, [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp]),
    "apus_hip_fp8_linear_dev": (C.c_int, [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp]),
    "apus_hip_store_create": (vp, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_size_t]),
    "apus_hip_store_free": (None, [vp]),
    "apus_hip_store_bytes": (C.c_uint64, [vp]),
    "apus_hip_store_fill_random": (C.c_int, [vp, C.c_uint64]),
    "apus_hip_store_put": (C.c_int, [vp, C.c_int, C.c_int, C.POINTER(ApusFp4W),
                                     C.POINTER(ApusFp4W), C.POINTER(ApusFp4W)]),
    "apus_hip_store_get": (C.c_int, [vp, C.c_int, C.c_int, C.POINTER(vp)]),
    "apus_hip_moe_workspace": (C.c_size_t, [vp, C.c_int, C.c_int]),
    "apus_hip_moe_routed_dev": (C.c_int, [vp, C.c_int, vp, vp, vp, C.c_int, C.c_int, C.c_float,
                                          vp, vp]),
    "apus_hip_moe_routed_dense_dev": (C.c_int, [vp, C.c_int, vp, vp, vp, C.c_int, C.c_int, C.c_float,
                                                vp, vp, vp, vp, C.c_int, vp]),
    "apus_hip_moe_noalloc_max": (C.c_size_t, []),
    "apus_hip_moe_routed_dev_noalloc": (C.c_int, [vp, C.c_int, vp, vp, vp, C.c_int, C.c_int,
                                                  C.c_float, vp]),
    "apus_hip_moe_routed_h": (C.c_int, [vp, C.c_int, C.c_int, vp, vp, vp]),
    "apus_hip_moe_forward_workspace": (C.c_size_t, [vp, C.c_int, C.c_int]),
    "apus_hip_moe_forward_dev": (C.c_int, [vp, C.c_int, C.POINTER(ApusHipMoeLayer), vp, vp,
                                           C.c_int, C.c_int, vp, C.POINTER(ApusHipMoeInterm),
                                           vp]),
    "apus_hip_container_open": (vp, [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_char_p,
                                     C.c_size_t]),
    "apus_hip_container_close": (None, [vp]),
    "apus_hip_container_slab": (C.c_int, [vp, C.c_int, C.c_int, C.POINTER(ApusHipSlabRec)]),
    "apus_hip_container_shard": (C.c_char_p, [vp, C.c_int]),
    "apus_hip_store_load": (C.c_int, [vp, vp, C.c_int, C.c_char_p, C.c_size_t]),
    "apus_hip_malloc": (vp, [C.c_size_t]),
    "apus_hip_free": (C.c_int, [vp]),
    "apus_hip_h2d": (C.c_int, [vp, vp, C.c_size_t]),
    "apus_hip_d2h": (C.c_int, [vp, vp, C.c_size_t]),
    "apus_hip_memset": (C.c_int, [vp, C.c_int, C.c_size_t]),
    "apus_hip_d2d": (C.c_int, [vp, vp, C.c_size_t]),
    "apus_hip_fill_random": (C.c_int, [vp, C.c_size_t, C.c_uint64, C.c_uint64, C.c_int]),
    "apus_hip_synchronize": (C.c_int, []),
    "apus_hip_timer_start": (C.c_int, []),
    "apus_hip_stream_delay": (C.c_int, [C.c_int]),
    "apus_hip_timer_stop": (C.c_float, []),
    "apus_hip_lanes": (C.c_int, [C.c_int]),
    "apus_hip_lane": (C.c_int, [C.c_int]),
    "apus_hip_fork": (C.c_int, []),
    "apus_hip_join": (C.c_int, []),
    "apus_hip_graph_begin": (C.c_int, []),
    "apus_hip_graph_end": (C.c_int, []),
    "apus_hip_graph_replay": (C.c_int, [C.c_int]),
    "apus_hip_last_error": (C.c_char_p, []),
    "apus_hip_device_info": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(C.c_int)]),
    "apus_hip_layer1": (C.c_int, [C.c_int, C.POINTER(C.c_uint)]),
    "apus_hip_layer1_spin_limit": (C.c_int, [C.c_uint]),
    "apus_hip_check_e4m3_hw": (C.c_int, [C.POINTER(C.c_uint), C.POINTER(C.c_uint)]),
    "apus_hip_host_bf16_round": (C.c_float, [C.c_float]),
    "apus_hip_host_e4m3_quant": (C.c_uint8, [C.c_float]),
    "apus_hip_host_act_scale": (C.c_float, [C.c_float]),
}

_lib = None


def lib():
    """Load libapus_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ApusHipError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc, what):
    if rc != 0:
        msg = lib().apus_hip_last_error().decode(errors="replace")
        raise ApusHipError(f"{what} failed: {msg}")


def _p(a, t):
    return a.ctypes.data_as(t)


def enable():
    buf = C.create_string_buffer(512)
    if lib().apus_hip_enable(buf, 512) != 0:
        raise ApusHipError("apus_hip_enable: " + buf.value.decode(errors="replace"))


def device_info():
    name = C.create_string_buffer(256)
    cus = C.c_int()
    _check(lib().apus_hip_device_info(name, 256, C.byref(cus)), "device_info")
    return name.value.decode(), cus.value


# ------------------------------------------------------------- host entry points

def act_quant(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    codes = np.empty((M, K), np.uint8)
    scales = np.empty((M, K // 128), np.float32)
    _check(lib().apus_hip_act_quant(_p(x, f32p), M, K, _p(codes, u8p), _p(scales, f32p)),
           "act_quant")
    return codes, scales


def fp4_gemm(w, ws, acodes, ascales):
    O = w.shape[0]
    M, K = acodes.shape
    out = np.empty((M, O), np.float32)
    _check(lib().apus_hip_fp4_gemm(_p(w, u8p), _p(ws, u8p), _p(acodes, u8p), _p(ascales, f32p),
                                   _p(out, f32p), M, O, K), "fp4_gemm")
    return out


def fp8_gemm(w, ws, acodes, ascales):
    O = w.shape[0]
    M, K = acodes.shape
    out = np.empty((M, O), np.float32)
    _check(lib().apus_hip_fp8_gemm(_p(w, u8p), _p(ws, u8p), _p(acodes, u8p), _p(ascales, f32p),
                                   _p(out, f32p), M, O, K), "fp8_gemm")
    return out


def fp4_weight(w, ws):
    return ApusFp4W(_p(w, u8p), _p(ws, u8p), w.shape[0], w.shape[1] * 2)


def fp8_weight(w, ws):
    return ApusFp8W(_p(w, u8p), _p(ws, u8p), w.shape[0], w.shape[1])


def fp4_linear(w, ws, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    O = w.shape[0]
    out = np.empty((M, O), np.float32)
    W = fp4_weight(w, ws)
    _check(lib().apus_hip_fp4_linear(C.byref(W), _p(x, f32p), _p(out, f32p), M, K, O),
           "fp4_linear")
    return out


def fp8_linear(w, ws, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    O = w.shape[0]
    out = np.empty((M, O), np.float32)
    W = fp8_weight(w, ws)
    _check(lib().apus_hip_fp8_linear(C.byref(W), _p(x, f32p), _p(out, f32p), M, K, O),
           "fp8_linear")
    return out


def f32_linear(w, x, flags=0):
    """Plain-weight linear hook: w [O, K] float32 (or uint16 BF16 bits with
    flags & 4), x [M, K] float32; flags 1 = BF16 input, 2 = BF16 output."""
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    O = w.shape[0]
    out = np.empty((M, O), np.float32)
    _check(lib().apus_hip_f32_linear(w.ctypes.data, _p(x, f32p), _p(out, f32p), M, K, O, flags),
           "f32_linear")
    return out


class StTensor(C.Structure):
    """c/st.h:46-53 ApusStTensor (head GEMV view)."""
    _fields_ = [("name", C.c_char * 160), ("dtype", C.c_int), ("ndim", C.c_int),
                ("shape", C.c_int64 * 8), ("data", vp), ("nbytes", C.c_size_t)]


def head_gemv(w, x):
    """LM-head GEMV over a BF16 (uint16 bits) or F32 view w [O, K]; x [K]."""
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    O, K = w.shape
    t = StTensor()
    t.name = b"head"
    t.dtype = 4 if w.dtype == np.uint16 else 6
    t.ndim = 2
    t.shape[0], t.shape[1] = O, K
    t.data = w.ctypes.data
    t.nbytes = w.nbytes
    out = np.empty(O, np.float32)
    _check(lib().apus_hip_head_gemv(C.byref(t), _p(x, f32p), _p(out, f32p), O, K), "head_gemv")
    return out


def fp4_gemm_grouped(entries, acodes, ascales, O):
    """entries: list of (w, ws, m0, M). Returns a list of [M, O] outputs."""
    K = acodes.shape[1]
    outs = [np.empty((M, O), np.float32) for (_, _, _, M) in entries]
    arr = (ApusFp4GemmEnt * len(entries))()
    for i, ((w, ws, m0, M), o) in enumerate(zip(entries, outs)):
        arr[i] = ApusFp4GemmEnt(_p(w, u8p), _p(ws, u8p), _p(o, f32p), m0, M)
    _check(lib().apus_hip_fp4_gemm_grouped(arr, len(entries), _p(acodes, u8p),
                                           _p(ascales, f32p), O, K), "fp4_gemm_grouped")
    return outs


def moe_routed(experts, x, idx, wgt, limit, layer_id=0, resolve=None, hint=None):
    """experts: list of E tuples (w1, w1s, w2, w2s, w3, w3s) of numpy arrays
    (w1/w3 [inter, dim/2], w2 [dim, inter/2]). x [s, dim]; idx/wgt [s, topk].

    resolve(layer, eid) -> a tuple like experts[eid] or None (failure), and
    hint(layer, eid), when given, are installed as ApusMoeW.hook_resolve /
    hook_hint (c/moe.h:45-56) and the w1/w2/w3 arrays are left NULL; the
    arrays a resolve returns must stay alive until the call returns."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    wgt = np.ascontiguousarray(wgt, dtype=np.float32)
    s, dim = x.shape
    topk = idx.shape[1]
    E = len(experts)
    inter = experts[0][0].shape[0]
    mw = ApusMoeW()
    mw.E, mw.topk, mw.inter, mw.dim = E, topk, inter, dim
    mw.limit = limit
    mw.layer_id = layer_id
    keep = []
    if resolve is None:
        a1 = (ApusFp4W * E)()
        a2 = (ApusFp4W * E)()
        a3 = (ApusFp4W * E)()
        for e, (w1, w1s, w2, w2s, w3, w3s) in enumerate(experts):
            a1[e] = ApusFp4W(_p(w1, u8p), _p(w1s, u8p), inter, dim)
            a2[e] = ApusFp4W(_p(w2, u8p), _p(w2s, u8p), dim, inter)
            a3[e] = ApusFp4W(_p(w3, u8p), _p(w3s, u8p), inter, dim)
        mw.w1, mw.w2, mw.w3 = a1, a2, a3
    else:
        def _resolve(ctx, layer, eid, p1, p2, p3):
            t = resolve(layer, eid)
            if t is None:
                return 1
            keep.append(t)
            w1, w1s, w2, w2s, w3, w3s = t
            p1[0] = ApusFp4W(_p(w1, u8p), _p(w1s, u8p), inter, dim)
            p2[0] = ApusFp4W(_p(w2, u8p), _p(w2s, u8p), dim, inter)
            p3[0] = ApusFp4W(_p(w3, u8p), _p(w3s, u8p), inter, dim)
            return 0
        mw.hook_resolve = RESOLVE_FN(_resolve)
        keep.append(mw.hook_resolve)
        if hint is not None:
            mw.hook_hint = HINT_FN(lambda ctx, layer, eid: hint(layer, eid))
            keep.append(mw.hook_hint)
    y = np.empty((s, dim), np.float32)
    _check(lib().apus_hip_moe_routed(C.byref(mw), _p(x, f32p), _p(idx, i32p), _p(wgt, f32p), s,
                                     _p(y, f32p)), "moe_routed")
    return y


# ----------------------------------------------------------- device memory helpers

class DevBuf:
    """A device allocation owned by Python (freed on close/del)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().apus_hip_malloc(self.nbytes)
        if not self.ptr:
            _check(1, f"apus_hip_malloc({nbytes})")

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        _check(lib().apus_hip_h2d(b.ptr, a.ctypes.data, a.nbytes), "h2d")
        return b

    def to_array(self, dtype, shape):
        out = np.empty(shape, dtype)
        _check(lib().apus_hip_d2h(out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def close(self):
        if self.ptr:
            lib().apus_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synchronize():
    _check(lib().apus_hip_synchronize(), "synchronize")
