"""The drop-in boundary on the CPU: the plugin-EP library, driven by a mock ORT host.

Covers what the reference tests without a GPU (rust/tests/mock_ort/mod.rs, rust/tests/
cdylib_load.rs, rust/src/ops/quant.rs unit tests): the exported symbols, ABI negotiation
(ORT_API_VERSION 28 down to 24, refusal below), the factory's identity, device advertisement
(none without a gfx950 device), the MatMulNBits claim predicate (quant.rs:110-203) and its
declines, the drop-constant-initializer decision, nested-graph declines, the claim allowlist,
Compile's out-slot contract on failure, and that every OrtStatus is released exactly once.
"""

from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import mock_host as mh
from oracle import matmul_nbits as orc

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / "include"


def _declared(header: Path) -> set[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b((?:mnb|Create|Release|OrtEpMi355x)\w*)\s*\(", text)) - {"CreateEpApiFactoriesFn"}


def _exported(so: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_libraries_export_every_declared_symbol():
    ep = _exported(mh.EP_SO)
    hip = _exported(ROOT / "onnxruntime-ep-vulkan_amd" / "lib" / "libmnb_hip.so")
    want_ep = _declared(INCLUDE / "onnxruntime_mi355x_ep.h")
    want_hip = _declared(INCLUDE / "mnb_hip.h")
    assert {"CreateEpFactories", "ReleaseEpFactory"} <= want_ep
    assert want_ep <= ep, want_ep - ep
    assert want_hip <= hip, want_hip - hip
    # the plugin exports nothing but its declared C surface
    assert {s for s in ep if not s.startswith("_")} == want_ep


@pytest.fixture
def host():
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0, "an OrtStatus was leaked"
    assert mh.lib().mock_bad_status_release() == 0, "an OrtStatus was released twice"


def test_factory_identity_and_negotiated_version(host):
    name, vendor, vid, ver = host.factory_info()
    assert name == "MI355XExecutionProvider"
    assert vid == 0x1002 and vendor
    assert ver == 28


@pytest.mark.parametrize("offered", [24, 25, 27])
def test_negotiates_down_to_the_host_version(offered):
    h = mh.Host(offered)
    assert h.init_rc == 0, mh.err()
    assert h.factory_info()[3] == offered
    assert h.close() == 0


def test_refuses_a_host_older_than_24():
    h = mh.Host(23)
    assert h.init_rc == mh.ORT_INVALID_ARGUMENT
    assert "ORT_API_VERSION >= 24" in h.init_error
    h.close()
    assert mh.lib().mock_live_statuses() == 0


def test_no_gfx950_device_advertises_nothing(host):
    # The CPU container has no GPU: zero devices, and no error (models fall back to the CPU EP).
    assert host.supported_devices(n_amd=1, n_other=1) == 0


def test_create_ep_rejects_several_devices(host):
    assert mh.lib().mock_create_ep_n(2) == mh.ORT_INVALID_ARGUMENT
    assert "one device per session" in mh.err()


def _graph(host, **over):
    """One MatMulNBits node (K=64, N=32, int4, bs=32, zp) with constant weights; `over` edits."""
    K, N, bits, bs = over.get("K", 64), over.get("N", 32), over.get("bits", 4), over.get("bs", 32)
    inp = orc.make_inputs(1, N, max(K, bs) - max(K, bs) % bs or bs, bits=bits, block_size=bs,
                          with_zp=True, seed=1)
    host.reset()
    el = mh.FLOAT16 if over.get("a_elem", mh.FLOAT16) == mh.FLOAT16 else over["a_elem"]
    host.value("A", el, over.get("a_shape", (1, K)))
    host.value("Y", el, (1, N))
    host.value("B", mh.UINT8, inp["B"].shape, None if over.get("b_input") else inp["B"])
    host.value("S", over.get("s_elem", el), inp["scales"].shape, inp["scales"])
    host.value("Z", over.get("z_elem", mh.UINT8), inp["zp"].shape, inp["zp"])
    host.value("G", mh.INT32, (K,), np.zeros(K, np.int32))
    host.value("BIAS", el, (N,), np.zeros(N, np.float16))
    ins = ["A", "B", "S", "Z"] + over.get("extra", [])
    attrs = {"K": K, "N": N, "bits": bits, "block_size": bs}
    if "acc" in over:
        attrs["accuracy_level"] = over["acc"]
    host.node(over.get("op", "MatMulNBits"), over.get("domain", "com.microsoft"), "mm", ins, ["Y"],
              attrs)


def test_claims_a_valid_node_and_drops_constant_weights(host):
    assert host.create_ep(-1) == 0
    assert mh.lib().mock_ep_name() == b"MI355XExecutionProvider"
    _graph(host)
    n, claimed = host.get_capability()
    assert n == 1 and claimed == ["mm:drop"]


@pytest.mark.parametrize("acc", [0, 1, 2, 3, 4])
def test_accuracy_levels_are_claimed(host, acc):
    # 0-3 resolve to ORT's fp32 path and are always claimed; 4 is claimed exactly when the HIP
    # library's planner implements the int8-activation kernel.
    import mnb
    assert host.create_ep(-1) == 0
    _graph(host, acc=acc)
    want = 1
    if acc == 4:
        try:
            mnb.plan(mnb.problem(1, 32, 64, 4, 32, True, mnb.DTYPE_F16, 4))
        except mnb.MnbError:
            want = 0
    assert host.get_capability()[0] == want


def test_accuracy_level_4_claim_follows_the_form(host):
    # the int8 path is int4 with block_size >= 32: level 4 at bits 8 or block 16 is declined
    assert host.create_ep(-1) == 0
    _graph(host, acc=4, bits=8)
    assert host.get_capability()[0] == 0
    _graph(host, acc=4, bs=16, K=64)
    assert host.get_capability()[0] == 0
    _graph(host, acc=4, bs=64, K=128)
    assert host.get_capability()[0] == 1


@pytest.mark.parametrize("case,over", [
    ("bits3", {"bits": 3}),
    ("bs256", {"bs": 256, "K": 512}),
    ("k_not_multiple", {"K": 48, "bs": 32}),
    ("g_idx", {"extra": ["G"]}),
    ("bias", {"extra": ["", "BIAS"]}),
    ("float_zero_points", {"z_elem": mh.FLOAT16}),
    ("int_activation", {"a_elem": mh.INT32}),
    ("scales_dtype_mismatch", {"s_elem": mh.FLOAT}),
    ("a_last_dim_not_k", {"a_shape": (1, 128)}),
    ("accuracy_level_5", {"acc": 5}),
    ("other_domain", {"domain": ""}),
    ("other_op", {"op": "MatMul"}),
])
def test_declines(host, case, over):
    assert host.create_ep(-1) == 0
    _graph(host, **over)
    n, claimed = host.get_capability()
    assert n == 0 and claimed == [], case


def test_symbolic_leading_dims_are_claimed(host):
    assert host.create_ep(-1) == 0
    _graph(host, a_shape=(-1, -1, 64))
    assert host.get_capability()[0] == 1


def test_non_constant_weights_are_kept(host):
    assert host.create_ep(-1) == 0
    _graph(host, b_input=True)
    assert host.get_capability()[1] == ["mm:keep"]


def test_keep_constant_initializers_option(host):
    host.option("ep.keep_constant_initializers", "1")
    assert host.create_ep(-1) == 0
    _graph(host)
    assert host.get_capability()[1] == ["mm:keep"]


def test_claim_allowlist_option(host):
    host.option("ep.max_claim_ops", "Gemm,MatMul")
    assert host.create_ep(-1) == 0
    _graph(host)
    assert host.get_capability()[0] == 0


def test_nested_subgraph_is_declined(host):
    assert host.create_ep(-1) == 0
    _graph(host)
    assert host.get_capability(nested=True)[0] == 0


def test_several_nodes_fuse_one_island_each(host):
    assert host.create_ep(-1) == 0
    host.reset()
    for i in range(3):
        inp = orc.make_inputs(1, 16, 64, seed=i)
        mh.add_matmul_nbits(host, f"n{i}", inp, 16, 64, 4, 32, (1, 64))
    n, claimed = host.get_capability()
    assert n == 3 and claimed == ["n0:drop", "n1:drop", "n2:drop"]


def test_compile_without_a_device_fails_cleanly(host):
    # No GPU here: Compile must return a status and leave every compute-info slot NULL.
    assert host.create_ep(-1) == 0
    _graph(host)
    assert host.get_capability()[0] == 1
    rc = host.compile()
    assert rc == mh.ORT_EP_FAIL, (rc, mh.err())
    assert "HIP" in mh.err() or "device" in mh.err()


# ---- device-memory mode (MI355X_EP_DEVICE_MEMORY; reference: rust/src/factory.rs:487-504) ----

@pytest.fixture
def dm_host(monkeypatch):
    # The factory reads the switch once, at CreateEpFactories.
    monkeypatch.setenv("MI355X_EP_DEVICE_MEMORY", "1")
    h = mh.Host(28)
    assert h.init_rc == 0, mh.err()
    yield h
    assert h.close() == 0
    assert mh.lib().mock_live_statuses() == 0
    assert mh.lib().mock_live_memory_infos() == 0, "the factory leaked an OrtMemoryInfo"


def test_stream_aware_only_in_device_memory_mode(dm_host):
    # IsStreamAware: host I/O has no stream to share; device-memory mode enqueues Compute on the
    # stream ORT creates through CreateSyncStreamForDevice (onnxruntime_ep_c_api.h)
    assert dm_host.is_stream_aware() == 1


def test_host_io_factory_is_not_stream_aware(host):
    assert host.is_stream_aware() == 0


def test_device_memory_is_off_by_default(host):
    # no allocator, no data transfer, no default memory device: ORT keeps every tensor on the host
    assert host.create_allocator_for(mh.MEM_GPU, mh.AMD, 0) == 0
    assert host.can_copy((mh.MEM_CPU, 0), (mh.MEM_GPU, mh.AMD)) == -1
    assert host.create_ep(-1) == 0, mh.err()
    assert host.default_memory_device()[0] == -2


@pytest.mark.parametrize("spelling", ["0", "off", "false", "no", "of", ""])
def test_device_memory_switch_fails_towards_host_io(monkeypatch, spelling):
    monkeypatch.setenv("MI355X_EP_DEVICE_MEMORY", spelling)
    h = mh.Host(28)
    try:
        assert h.create_allocator_for(mh.MEM_GPU, mh.AMD, 0) == 0
    finally:
        assert h.close() == 0


def test_device_allocator_serves_only_its_own_memory(dm_host):
    assert dm_host.create_allocator_for(mh.MEM_GPU, mh.AMD, 0) == 1
    assert dm_host.create_allocator_for(mh.MEM_GPU, mh.AMD, 3) == 1
    assert dm_host.create_allocator_for(mh.MEM_CPU, 0, 0) == 0
    assert dm_host.create_allocator_for(mh.MEM_GPU, mh.NVIDIA, 0) == 0
    assert dm_host.create_allocator_for(mh.MEM_GPU, mh.AMD, 0, mem=5) == 0   # HOST_ACCESSIBLE


def test_data_transfer_copies_host_and_hbm_only(dm_host):
    host_, amd, nv = (mh.MEM_CPU, 0), (mh.MEM_GPU, mh.AMD), (mh.MEM_GPU, mh.NVIDIA)
    assert dm_host.can_copy(host_, amd) == 1
    assert dm_host.can_copy(amd, host_) == 1
    assert dm_host.can_copy(amd, amd) == 1
    assert dm_host.can_copy(host_, host_) == 0
    assert dm_host.can_copy(nv, host_) == 0
    assert dm_host.can_copy(host_, nv) == 0


def test_default_memory_device_is_the_eps_hbm(dm_host, monkeypatch):
    dm_host.option("ep.device_index", 2)
    assert dm_host.create_ep(-1) == 0, mh.err()
    r, (t, vendor, dev) = dm_host.default_memory_device()
    assert r == 1 and t == mh.MEM_GPU and vendor == mh.AMD and dev == 2
