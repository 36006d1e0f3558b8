"""Expert slabs from an apus container into the HBM store
(apus_hip_store_load).

Every expert read back from the store (unpacked when the store holds the
MFMA-tiled layout) equals the tensors written into the container byte for
byte, and the routed dispatch over the loaded store matches the oracle on
those experts (bar 2^-7, as for the store-filled tests). A container whose
shapes do not match the store is refused before anything is read.
"""
import ctypes as C

import numpy as np
import pytest

import container_util as cu
from helpers import acts, max_rel, topk_routing
from test_gpu_store import read_expert

pytestmark = pytest.mark.gpu


def open_container(hip, path, n_layers, n_mtp, E):
    err = C.create_string_buffer(512)
    c = hip.lib().apus_hip_container_open(str(path).encode(), n_layers, n_mtp, E, err, 512)
    assert c, err.value
    return c


@pytest.mark.parametrize("dim,inter,E,n_mtp,threads", [(256, 128, 6, 1, 3), (2048, 2048, 4, 0, 0)])
def test_store_load_roundtrip_and_dispatch(hip, oracle, tmp_path, rng, dim, inter, E, n_mtp, threads):
    n_layers = 2 + n_mtp
    experts, shards, k = {}, {"s1.safetensors": [], "s2.safetensors": []}, 0
    for layer in range(n_layers):
        mtp = layer >= 2
        for e in range(E):
            experts[(layer, e)] = cu.expert_arrays(rng, dim, inter)
            order = [int(v) for v in rng.permutation(6)]
            shards["s1.safetensors" if k % 2 else "s2.safetensors"].extend(
                cu.expert_entries(layer - 2 if mtp else layer, e, experts[(layer, e)], mtp, order))
            k += 1
    cu.write_container(str(tmp_path), shards)
    L = hip.lib()
    c = open_container(hip, tmp_path, n_layers, n_mtp, E)
    err = C.create_string_buffer(256)
    st = L.apus_hip_store_create(n_layers, E, dim, inter, err, 256)
    assert st, err.value
    try:
        lerr = C.create_string_buffer(512)
        assert L.apus_hip_store_load(st, c, threads, lerr, 512) == 0, lerr.value
        for (layer, e), arr in experts.items():
            back = read_expert(hip, st, layer, e, dim, inter)
            for a, b in zip(arr, back):
                assert np.array_equal(a, b), (layer, e)
        # the routed dispatch over the loaded store, last layer (an MTP layer
        # when there is one)
        layer, s, topk = n_layers - 1, 3, min(4, E)
        x = acts(rng, s, dim)
        idx, wgt = topk_routing(rng, s, E, topk)
        want = oracle.moe_routed([experts[(layer, e)] for e in range(E)], x, idx, wgt, 10.0)
        dx, di, dw = (hip.DevBuf.from_array(a) for a in (x, idx, wgt))
        dy = hip.DevBuf(s * dim * 4)
        wsp = hip.DevBuf(L.apus_hip_moe_workspace(st, s, topk))
        hip._check(L.apus_hip_moe_routed_dev(st, layer, dx.ptr, di.ptr, dw.ptr, s, topk, 10.0,
                                             dy.ptr, wsp.ptr), "moe_routed_dev")
        got = dy.to_array(np.float32, (s, dim))
        assert max_rel(got, want) <= 2.0 ** -7
    finally:
        L.apus_hip_store_free(st)
        L.apus_hip_container_close(c)


def test_store_load_refuses_other_shapes(hip, tmp_path, rng):
    arr = cu.expert_arrays(rng, 256, 128)
    cu.write_container(str(tmp_path), {"s.safetensors": cu.expert_entries(0, 0, arr)})
    L = hip.lib()
    c = open_container(hip, tmp_path, 1, 0, 1)
    err = C.create_string_buffer(256)
    st = L.apus_hip_store_create(1, 1, 512, 128, err, 256)
    assert st, err.value
    try:
        lerr = C.create_string_buffer(512)
        assert L.apus_hip_store_load(st, c, 2, lerr, 512) != 0
        assert b"the store holds" in lerr.value
    finally:
        L.apus_hip_store_free(st)
        L.apus_hip_container_close(c)
