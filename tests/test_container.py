"""apus container index (apus_hip_container_*), host only.

The index must equal the reference expert store's own slab records
(c/cache.h apus_store_open, compiled from the apus sources in
oracle/_ref) on the same synthetic containers — shard, offset, length,
member offsets and shapes — and fail where the reference fails:
a missing member, an expert split across shards, a gap inside a slab, a
dtype or shape mismatch, slabs of different sizes. The containers are
written by tests/container_util.py in the format of c/st.h:5-10.
"""
import ctypes as C

import numpy as np
import pytest

import container_util as cu

E, DIM, INTER = 4, 256, 128


def lib_index(path, n_layers, n_mtp, n_experts):
    import apus_hip
    L = apus_hip.lib()
    err = C.create_string_buffer(512)
    c = L.apus_hip_container_open(path.encode(), n_layers, n_mtp, n_experts, err, 512)
    if not c:
        raise ValueError(err.value.decode())
    try:
        out = []
        rec = apus_hip.ApusHipSlabRec()
        for i in range(n_layers * n_experts):
            assert L.apus_hip_container_slab(c, i // n_experts, i % n_experts, C.byref(rec)) == 0
            out.append((L.apus_hip_container_shard(c, rec.shard).decode(), rec.off, rec.len,
                        list(rec.rel), list(rec.O), list(rec.K)))
        assert L.apus_hip_container_slab(c, n_layers, 0, C.byref(rec)) != 0
        assert L.apus_hip_container_shard(c, 10 ** 6) is None
        return out
    finally:
        L.apus_hip_container_close(c)


def build(tmp_path, rng, n_main=2, n_mtp=0, layout="plain", subdir=False):
    """A container of n_main + n_mtp expert layers with E experts each.
    layouts: plain (one shard, canonical order); spread (experts over three
    shards, dense tensors between slabs, members permuted inside slabs)."""
    experts = {}
    shards = {"model-00001.safetensors": [], "model-00002.safetensors": [],
              "model-00003.safetensors": []}
    names = list(shards)
    k = 0
    for layer in range(n_main + n_mtp):
        mtp = layer >= n_main
        for e in range(E):
            arr = cu.expert_arrays(rng, DIM, INTER)
            experts[(layer, e)] = arr
            order = range(6)
            if layout == "spread":
                order = [int(v) for v in rng.permutation(6)]
                shards[names[k % 3]].append(cu.dense_entry(f"layers.{layer}.attn.w{k}", rng,
                                                            200 + 64 * k))
            entries = cu.expert_entries(layer - n_main if mtp else layer, e, arr, mtp, order)
            shards[names[k % 3] if layout == "spread" else names[0]].extend(entries)
            k += 1
    shards = {n: v for n, v in shards.items() if v}
    d = cu.write_container(str(tmp_path), shards, subdir=subdir)
    return d, experts


@pytest.mark.parametrize("layout,n_mtp,subdir", [("plain", 0, False), ("spread", 0, True),
                                                 ("spread", 1, False)])
def test_index_equals_reference_store(tmp_path, rng, ref, layout, n_mtp, subdir):
    _, experts = build(tmp_path, rng, 2, n_mtp, layout, subdir)
    n_layers = 2 + n_mtp
    got = lib_index(str(tmp_path), n_layers, n_mtp, E)
    want, slabs = ref.store_index(str(tmp_path), n_layers, n_mtp, E, with_slabs=True)
    assert got == want
    # the records address the expert's bytes: reading them back gives the
    # tensors that were written, and the reference store reads the same slab
    d = str(tmp_path / "weights") if subdir else str(tmp_path)
    for i, (shard, off, ln, rel, O, K) in enumerate(got):
        with open(f"{d}/{shard}", "rb") as f:
            f.seek(off)
            blob = np.frombuffer(f.read(ln), np.uint8)
        assert np.array_equal(blob, slabs[i, :ln])
        arr = experts[(i // E, i % E)]
        for j in range(6):
            a = arr[j].ravel()
            assert np.array_equal(blob[rel[j]:rel[j] + a.size], a)
        assert O == [INTER, DIM, INTER] and K == [DIM, INTER, DIM]


def test_index_skips_layers_and_experts_outside_the_store(tmp_path, rng, ref):
    """Experts beyond n_experts and main layers at or past n_main are not
    indexed; the remaining ones must still be complete."""
    build(tmp_path, rng, 3, 0, "plain")
    got = lib_index(str(tmp_path), 2, 0, 3)
    want, _ = ref.store_index(str(tmp_path), 2, 0, 3)
    assert got == want


def corrupt(tmp_path, rng, how):
    arrs = [cu.expert_arrays(rng, DIM, INTER) for _ in range(2)]
    a0 = cu.expert_entries(0, 0, arrs[0])
    a1 = cu.expert_entries(0, 1, arrs[1])
    shards = {"a.safetensors": a0 + a1}
    extra = None
    if how == "missing":
        shards["a.safetensors"] = a0 + a1[:5]
    elif how == "split":
        shards = {"a.safetensors": a0 + a1[:3], "b.safetensors": a1[3:]}
    elif how == "gap":
        shards["a.safetensors"] = a0 + a1[:2] + [cu.dense_entry("gap.t", rng)] + a1[2:]
    elif how == "dtype":
        n, _, shp, data = a1[1]
        a1[1] = (n, "U8", shp, data)
        shards["a.safetensors"] = a0 + a1
    elif how == "slab_size":
        small = cu.expert_arrays(rng, DIM, INTER // 2)
        shards["a.safetensors"] = a0 + cu.expert_entries(0, 1, small)
    elif how == "absent_tensor":
        shards["a.safetensors"] = a0 + a1[:5]
        extra = {a1[5][0]: "a.safetensors"}
    cu.write_container(str(tmp_path), shards, extra_map=extra)


@pytest.mark.parametrize("how", ["missing", "split", "gap", "dtype", "slab_size", "absent_tensor"])
def test_index_rejects_what_the_reference_rejects(tmp_path, rng, ref, how):
    corrupt(tmp_path, rng, how)
    with pytest.raises(ValueError) as r_err:
        ref.store_index(str(tmp_path), 1, 0, 2)
    with pytest.raises(ValueError) as g_err:
        lib_index(str(tmp_path), 1, 0, 2)
    key = {"missing": "tensors in weight_map", "split": "split across shards",
           "gap": "not contiguous", "dtype": "shape/dtype mismatch", "slab_size": "slab",
           "absent_tensor": "missing tensor"}[how]
    assert key in str(r_err.value) and key in str(g_err.value), (r_err.value, g_err.value)


def test_index_name_rules(tmp_path, rng):
    """Only canonical expert names count: suffix garbage, leading zeros,
    signs and w0/w4 are ignored (c/cache.h:381-407), so the expert stays
    incomplete."""
    arr = cu.expert_arrays(rng, DIM, INTER)
    good = cu.expert_entries(0, 0, arr)
    bad_names = ["layers.0.ffn.experts.0.w1.weightx", "layers.00.ffn.experts.0.w1.weight",
                 "layers.+0.ffn.experts.0.w1.weight", "layers.0.ffn.experts.0.w4.weight"]
    for bn in bad_names:
        entries = [(bn, "I8", good[0][2], good[0][3])] + good[1:]
        d = tmp_path / bn.replace("+", "p")
        d.mkdir()
        cu.write_container(str(d), {"s.safetensors": entries})
        with pytest.raises(ValueError, match="5/6 tensors"):
            lib_index(str(d), 1, 0, 1)
