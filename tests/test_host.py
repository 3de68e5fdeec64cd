"""CPU tests of the host side: the C ABI library (loads, exports, validates
arguments without touching a GPU), the schedule, and product/oracle
separation."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from oracle import kvm_oracle as O

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvm_amd.h"


def _lib():
    from kvm_amd import _lib

    try:
        return _lib.load()
    except _lib.KvmLibraryError as e:  # not built in this checkout
        pytest.skip(str(e))


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvm_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib()
    names = _declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), f"libkvm_amd.so does not export {n}"
    from kvm_amd import _lib as L

    assert set(names) == set(L.SIGNATURES), "binding and header disagree"


def test_struct_layout_matches_binding():
    lib = _lib()
    from kvm_amd import _lib as L

    assert lib.kvm_abi_version() == L.ABI_VERSION
    for i, st in enumerate((L.KvmLayer, L.KvmSeq, L.KvmState, L.KvmPrefillDesc, L.KvmPrefixDesc, L.KvmPrefillBwdDesc,
                              L.KvmStateBwdDesc, L.KvmAddNormDesc)):
        assert lib.kvm_struct_size(i) == ctypes.sizeof(st)
    assert lib.kvm_struct_size(9) == -1


def test_header_abi_version_matches_binding():
    from kvm_amd import _lib as L

    m = re.search(r"#define KVM_ABI_VERSION (\d+)", HEADER.read_text())
    assert m and int(m.group(1)) == L.ABI_VERSION
    for name in ("KVM_EABORT", "KVM_STATUS_CHAIN_TIMEOUT"):
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", HEADER.read_text())
        assert m and int(m.group(1)) == getattr(L, name)


def test_integration_stub_binds_the_library(monkeypatch):
    """The ctypes stub printed in INTEGRATION.md section 3 runs against the
    built library: its ABI assert, struct-size asserts and argument list."""
    _lib()
    from kvm_amd import _lib as L

    text = (ROOT / "INTEGRATION.md").read_text()
    sec = text[text.index("## 3. Binding the C ABI directly"):]
    block = sec[sec.index("```python") + len("```python"):]
    block = block[:block.index("```")]
    monkeypatch.setenv("LIBKVM_AMD", str(L.LIB_PATH))
    ns: dict = {}
    exec(compile(block, "INTEGRATION.md:stub", "exec"), ns)
    lib = ns["lib"]
    assert ns["KVM_ABI_VERSION"] == L.ABI_VERSION
    assert ctypes.sizeof(ns["KvmLayer"]) == ctypes.sizeof(L.KvmLayer)
    assert ctypes.sizeof(ns["KvmState"]) == ctypes.sizeof(L.KvmState)
    assert len(lib.kvm_decode_attention.argtypes) == len(L.SIGNATURES["kvm_decode_attention"][1])
    assert callable(ns["kvm_decode_attention"])


def _layer(**kw):
    from kvm_amd import _lib as L

    w = torch.ones(128)
    base = dict(batch=1, q_heads=4, kv_heads=2, head_dim=128, value_dim=128, chunk_len=64, n_bswa_chunks=2,
                sink_len=1, rope_partial_dim=32, gate_keys=1, gate_values=1, gate_appends=0, gate_initial=0,
                ln_eps=1e-5, ln_weight=w.data_ptr(), ln_bias=w.data_ptr(), state_temp=w.data_ptr(),
                front_temp=w.data_ptr())
    base.update(kw)
    return L.KvmLayer(**base), w


@pytest.mark.parametrize("field,value,msg", [
    ("head_dim", 96, "head_dim"),
    ("value_dim", 64, "value_dim"),
    ("q_heads", 3, "multiple of kv_heads"),
    ("chunk_len", 0, "chunk_len"),
    ("rope_partial_dim", 200, "rope_partial_dim"),
    ("ln_eps", 0.0, "ln_eps"),
])
def test_invalid_layer_is_rejected_before_any_gpu_work(field, value, msg):
    lib = _lib()
    from kvm_amd import _lib as L

    layer, keep = _layer(**{field: value})
    st = L.KvmState(16, 16, 16, 16, 16, 8)
    rc = lib.kvm_state_refresh(ctypes.byref(layer), ctypes.byref(st), 0, 1, None)
    assert rc == L.KVM_EINVAL
    assert msg in lib.kvm_last_error().decode()
    with pytest.raises(ValueError):
        L.check(rc, "refresh")


def test_decode_step_argument_checks():
    """kvm_decode_step refuses, before any GPU work, a token taken from a
    ring, a missing gate ring and a window that does not hold the token."""
    lib = _lib()
    from kvm_amd import _lib as L

    layer, keep = _layer()
    st = L.KvmState(16, 16, 16, 16, 16, 8)

    def call(seq, ring_gate=16, recent_len=1):
        return lib.kvm_decode_step(ctypes.byref(layer), 16, 8, 8, ctypes.byref(st), 0, ctypes.byref(seq), 16, 16,
                                   ring_gate, 8, 0, recent_len, 16, 8, 8, 16, 1 << 30, None)

    plain = L.KvmSeq(16, 16, 16, 8, 8, 8, 8, 8, 8, 1, 1, 1, 0)
    ringed = L.KvmSeq(16, 16, 16, 8, 8, 8, 8, 8, 8, 1, 1, 1, 4)
    assert call(ringed) == L.KVM_EINVAL and "ring" in lib.kvm_last_error().decode()
    assert call(plain, ring_gate=None) == L.KVM_EINVAL and "ring_gate" in lib.kvm_last_error().decode()
    assert call(plain, recent_len=0) == L.KVM_EINVAL and "last window row" in lib.kvm_last_error().decode()
    assert call(plain, recent_len=9) == L.KVM_EINVAL and "outside the ring" in lib.kvm_last_error().decode()


def test_add_norm_rejects_aliased_outputs():
    """kvm_add_norm refuses, before any GPU work, an output that is x or y
    when seq_len > 1 (the token shift reads the previous run's last row,
    which an aliased output may already have overwritten); one token may be
    updated in place."""
    lib = _lib()
    from kvm_amd import _lib as L

    def call(seq_len, **out):
        d = L.KvmAddNormDesc()
        d.x, d.y, d.alpha, d.ln_w, d.ln_b, d.eps = 16, 32, 1.0, 48, 64, 1e-5
        d.mix, d.prev = 80, 96
        d.batch, d.seq_len, d.width = 2, seq_len, 128
        for k, v in out.items():
            setattr(d, k, v)
        return lib.kvm_add_norm(ctypes.byref(d), None)

    for field, ptr in (("out_x", 16), ("out_h", 32), ("out_shift", 16)):
        assert call(8, **{field: ptr}) == L.KVM_EINVAL, field
        assert "alias x or y" in lib.kvm_last_error().decode()
    assert call(8, out_x=112, out_h=128, out_shift=144, state_out=96) == L.KVM_EINVAL
    assert "state_out may alias prev" in lib.kvm_last_error().decode()


def test_update_argument_checks():
    lib = _lib()
    from kvm_amd import _lib as L

    layer, keep = _layer(sink_len=4)
    seq = L.KvmSeq(16, 16, 16, 8, 8, 8, 8, 8, 8, 1, 1, 1, 0)
    st = L.KvmState(16, 16, 16, 16, 16, 4)
    args = lambda before, n_app, ws: (ctypes.byref(layer), ctypes.byref(seq), 0, 64, before, n_app, ctypes.byref(st),
                                      16, 16, 16, ws, None, None, None)
    # Every slot is a sink: merging is impossible (model/kvm_mixer.py:309-314).
    assert lib.kvm_state_update(*args(4, 0, 1 << 30)) == L.KVM_EINVAL
    assert "non-sink" in lib.kvm_last_error().decode()
    # State grows past the capacity.
    assert lib.kvm_state_update(*args(2, 8, 1 << 30)) == L.KVM_ESPACE
    # Workspace too small.
    st.capacity = 100
    layer.sink_len = 1
    assert lib.kvm_state_update(*args(10, 0, 16)) == L.KVM_ESPACE
    assert "workspace" in lib.kvm_last_error().decode()
    # Misaligned pointers.
    seq.k = 18
    assert lib.kvm_state_update(*args(10, 0, 1 << 30)) == L.KVM_EINVAL
    assert "aligned" in lib.kvm_last_error().decode()


def test_workspace_queries():
    lib = _lib()
    layer, keep = _layer()
    n = lib.kvm_update_workspace_bytes(ctypes.byref(layer), 64)
    rows = 2
    assert n >= 3 * rows * 64 * 128 * 2 + 3 * rows * 64 * 4
    assert lib.kvm_decode_workspace_bytes(ctypes.byref(layer), 1000) == 1 * 4 * 4 * (128 + 2) * 4
    bad, keep2 = _layer(head_dim=80)
    assert lib.kvm_update_workspace_bytes(ctypes.byref(bad), 64) == -1


def test_prefill_schedule_validation():
    lib = _lib()
    from kvm_amd import _lib as L
    from kvm_amd.schedule import StateBudget, prefill_plan

    layer, keep = _layer(chunk_len=64)
    plan = prefill_plan(1000, 64, 2, StateBudget("fixed", 1.0, 0.5, 1, 64, None, 64))
    d = L.KvmPrefillDesc()
    d.layer = layer
    d.q, d.q_sb, d.q_sh, d.q_st = 16, 8, 8, 8
    d.kv = L.KvmSeq(16, 16, 16, 8, 8, 8, 8, 8, 8, 1, 1, 1, 0)
    d.seq_len = 1000
    d.out, d.o_sb, d.o_st, d.o_sh = 16, 8, 8, 8
    d.state = L.KvmState(16, 16, 16, 16, 16, 64)
    arrs = [L.int32_array(a) for a in (plan.chunk_state_len, plan.chunk_snapshot, plan.upd_token_begin,
                                        plan.upd_state_before, plan.upd_n_append)]
    d.n_chunks = plan.n_chunks
    d.chunk_state_len, d.chunk_snapshot = arrs[0], arrs[1]
    d.n_updates = plan.n_updates
    d.upd_token_begin, d.upd_state_before, d.upd_n_append = arrs[2], arrs[3], arrs[4]
    d.max_state_len = plan.max_state_len
    d.snapshot_ring = 4
    need = lib.kvm_prefill_workspace_bytes(ctypes.byref(d))
    assert need > 0
    d.workspace, d.workspace_bytes = 16, need - 1
    assert lib.kvm_prefill(ctypes.byref(d), None) == L.KVM_ESPACE
    d.workspace_bytes = need
    d.n_chunks = plan.n_chunks + 1
    assert lib.kvm_prefill(ctypes.byref(d), None) == L.KVM_EINVAL
    d.n_chunks = plan.n_chunks
    arrs[3][2] += 1  # inconsistent state lengths
    assert lib.kvm_prefill(ctypes.byref(d), None) == L.KVM_EINVAL
    assert "starts from" in lib.kvm_last_error().decode()


# --------------------------------------------------------------------------
# Schedule: product restatement vs oracle, closed forms of the BASELINE configs.

CASES = [
    (32768, 512, 2, ("fixed", 1.0, 0.5, 1, 256, None, 512)),
    (65536, 512, 2, ("power_law", 1.0, 0.5, 1, -1, None, 1024)),
    (65536, 512, 2, ("power_law", 16.0, 0.5, 1, -1, None, 1024)),
    (4096, 256, 2, ("fixed", 1.0, 0.5, 1, 64, None, 256)),
    (1100, 64, 2, ("power_law", 5.0, 0.5, 1, 64, None, 192)),
    (777, 64, 3, ("kvm_saturation", 1.0, 0.5, 8, 16, 300, 256)),
    (20, 32, 2, ("fixed", 1.0, 0.5, 1, 32, None, 32)),
]


@pytest.mark.parametrize("T,C,n,budget", CASES)
def test_plan_matches_oracle_schedule(T, C, n, budget):
    from kvm_amd.schedule import StateBudget, prefill_plan

    mode, f, e, rd, mn, sat, mx = budget
    b = StateBudget(mode, f, e, rd, mn, sat, mx)
    plan = prefill_plan(T, C, n, b)
    cfg = O.OracleConfig(q_heads=1, kv_heads=1, head_dim=64, value_dim=64, chunk_len=C, n_bswa_chunks=n,
                         n_max_d_chunks=mx // C, state_budget_mode=mode, state_growth_factor=f,
                         state_growth_exponent=e, state_round_down=rd, state_min_len=mn, state_saturation_n=sat)
    ref = O.prefill_schedule(cfg, T)
    assert plan.front_len == ref["front_len"]
    assert plan.final_state_len == ref["final_state_len"]
    assert plan.final_coverage == ref["final_coverage"]
    assert [(tb // C, c, a, bf, bf + na, na) for tb, c, a, bf, na in
            zip(plan.upd_token_begin, plan.upd_ctx_len, plan.upd_available, plan.upd_state_before,
                plan.upd_n_append)] == ref["updates"]
    for m, s in ref["attention_state_len"].items():
        assert plan.chunk_state_len[m] == s
        # chunk m >= n sees the state after the m - n updates before it
        assert plan.chunk_snapshot[m] == m - n


def test_baseline_config_closed_forms():
    from kvm_amd.schedule import StateBudget, prefill_plan

    # config 2: state floor = first chunk (512 slots), 61 updates, coverage 31744
    p = prefill_plan(32768, 512, 2, StateBudget("fixed", 1.0, 0.5, 1, 256, None, 512))
    assert (p.n_updates, p.final_state_len, p.final_coverage) == (61, 512, 31744)
    # config 3, literal floor(sqrt(t)) growth never passes the 512 floor
    p = prefill_plan(65536, 512, 2, StateBudget("power_law", 1.0, 0.5, 1, -1, None, 1024))
    assert (p.n_updates, p.final_state_len) == (125, 512) and sum(p.upd_n_append) == 0
    # config 3 with f = 16: floor(16 sqrt(t)) reaches the 1024 cap
    p = prefill_plan(65536, 512, 2, StateBudget("power_law", 16.0, 0.5, 1, -1, None, 1024))
    assert p.final_state_len == 1024 and p.max_state_len == 1024


def test_benchmark_harness_schedule_helpers():
    """The helpers the reference's benchmark harness calls on the mixer
    (scripts/kvm_benchmark/common.py:153-155) give the state length of the
    schedule, for fixed and growable budgets."""
    import bench
    from kvm_amd import SequenceMixer

    cfg = bench._config(32, 32, 128, 512, 2, 256, 1)
    m = SequenceMixer(cfg, 0)
    args = m._make_triton_args(8, 32768)
    assert (args.q_len, args.logical_q_len, args.initial_state_len) == (32768, 32768, 512)
    assert m._make_schedule(args).final_state_len == 512
    cfg = bench._config(16, 16, 128, 512, 2, -1, 2)
    cfg.state_budget_mode, cfg.state_growth_factor = "power_law", 16.0
    m = SequenceMixer(cfg, 0)
    # 1000 tokens pad to two chunks; the schedule follows the logical length
    assert m._make_triton_args(2, 1000).q_len == 1024
    assert m._make_schedule(m._make_triton_args(2, 65536)).final_state_len == 1024


def test_bench_flop_count_matches_brute_force():
    import bench
    from kvm_amd.schedule import StateBudget, prefill_plan

    for T, C, n in ((777, 64, 2), (1000, 128, 3), (64, 64, 2)):
        plan = prefill_plan(T, C, n, StateBudget("power_law", 6.0, 0.5, 1, C, None, 3 * C))
        brute = 0
        for t in range(T):
            m = t // C
            wb = max(0, (m - n + 1) * C)
            brute += plan.chunk_state_len[m] + (t - wb + 1)
        assert bench.attention_pairs(plan, n) == brute


def test_product_never_imports_the_oracle():
    pkg = ROOT / "kvm-paper_amd"
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.hpp")):
        text = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, flags=re.M), f"{f} imports the oracle"
        assert "kvm_oracle" not in text, f"{f} references the oracle"


@pytest.mark.parametrize("src", ["kvm_attn.hip", "kvm_chain.hip"])
def test_m0_only_written_by_the_lds_dma_helpers(src, tmp_path):
    """The inline-assembly LDS-DMA loads set M0 without declaring it clobbered
    (the compiler rejects M0 as a clobber); that is sound only while the
    compiled kernels use M0 for nothing else.  Compile the device code and
    check that every M0 write is one of those statements, immediately followed
    by its buffer load into LDS."""
    import shutil
    import subprocess

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / "k.s"
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        "-o", str(out), str(ROOT / "kvm-paper_amd" / "csrc" / src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln.strip() for ln in out.read_text().splitlines()]
    code = [ln for ln in lines if ln and not ln.startswith((";", "."))]
    writes = 0
    for i, ln in enumerate(code):
        if re.search(r"\bm0\b", ln):
            assert re.fullmatch(r"s_mov_b32 m0, s\d+", ln), f"{src}: unexpected use of M0: {ln}"
            nxt = code[i + 1]
            assert nxt.startswith("buffer_load_dwordx4") and nxt.endswith(" lds"), (src, ln, nxt)
            writes += 1
    assert writes > 0


def test_torch_operator_library_registers_the_ops():
    """libkvm_amd_torch.so (csrc/kvm_torch_ops.cpp) loads over the C library
    and registers torch.ops.kvm_amd.prefill / decode_step with schemas that
    mark their outputs as written."""
    _lib()
    import torch
    from kvm_amd import _lib as L

    ops = L.ops()
    prefill = str(ops.prefill.default._schema)
    decode = str(ops.decode_step.default._schema)
    assert prefill.startswith("kvm_amd::prefill(") and "Tensor(a!) out" in prefill and "int[] cfg" in prefill
    assert decode.startswith("kvm_amd::decode_step(") and "Tensor(d!) out" in decode
    assert torch.ops.kvm_amd.prefill is ops.prefill
