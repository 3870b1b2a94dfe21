"""The hc kernel-definition and launch surface (host logic, no GPU).

Mirrors the reference's public-API and simulator-binding tests
(tests/test_public_api.py:26-114, tests/test_simulator.py:170-208) for what
the gfx950 target keeps: decorator metadata, Buffer specs, intrinsic hooks,
symbol binding with conflict detection, geometry validation, error classes,
and the zero-size no-op.
"""

from __future__ import annotations

import numpy as np
import pytest

import hc
import hc.gfx950 as g
from hc import Buffer, LaunchError, SimulatorError, WorkItem, kernel, sym
from hc._launch import prepare_launch
from hc.simulator import SimulatorTarget
from hc.symbols import Bindings, SymbolConflictError, ceil_div

from . import _kernels


def test_public_names_match_reference_list():
    for name in ["Buffer", "BufferSpec", "CompiledKernel", "CurrentGroup", "IdxTypeSpec", "IndexMap",
                 "Result", "Scope", "SubGroup", "Symbol", "TensorTypeSpec", "UndefTypeSpec",
                 "VectorTypeSpec", "WorkGroup", "WorkItem", "as_layout", "compile", "idx_type",
                 "index_map", "kernel", "simulator", "sym", "symbols", "tensor_type", "undef_type",
                 "vector_type"]:
        assert hasattr(hc, name), name


def test_kernel_decorator_attaches_metadata_and_returns_function():
    def f(group, x: Buffer[sym.M, np.float16]):
        pass

    out = kernel(work_shape=(sym.M,), group_shape=(64,), subgroup_size=64, literals={sym.M})(f)
    assert out is f
    md = f.__hc_kernel__
    assert md.work_shape == (sym.M,) and md.group_shape == (64,) and md.subgroup_size == 64
    assert md.literals == frozenset({sym.M})


def test_buffer_spec_forms():
    spec = Buffer[sym.M, sym.K, np.float16]
    assert spec.dimensions == (sym.M, sym.K) and spec.dtype == "float16"
    assert Buffer[sym.M].dtype is None
    assert Buffer[sym.M, hc.bfloat16].dtype == "bfloat16"
    assert Buffer[sym.M, np.dtype(np.float32)].dtype == "float32"
    assert repr(Buffer[sym.M, 4, np.float32]) == "Buffer[M, 4, float32]"


def test_intrinsic_hooks_and_fallback_detection():
    @kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"arch"}, result_types=hc.idx_type())
    def with_body(x, *, arch):
        return x + 1

    @kernel.intrinsic(scope=WorkItem)
    def bodyless(x):
        """Doc only."""

    @kernel.intrinsic(scope=WorkItem)
    def ellipsis(x):
        ...

    assert with_body.__hc_has_fallback__ and not bodyless.__hc_has_fallback__
    assert not ellipsis.__hc_has_fallback__
    assert with_body.__hc_intrinsic__.const_attrs == frozenset({"arch"})
    assert with_body.__hc_intrinsic__.result_types == (hc.idx_type(),)

    @with_body.lower(target="amdgpu-gfx950")
    def _lower(ctx, x, *, arch):
        return None

    @with_body.verify
    def _verify(sig, target):
        return None

    assert with_body.__hc_lowerings__ == {"amdgpu-gfx950": _lower}
    assert with_body.__hc_verify__ is _verify


def test_gfx950_example_kernel_registers_its_intrinsic_lowering():
    from hc.gfx950 import kernels

    assert "amdgpu-gfx950" in kernels.mfma_gfx950.__hc_lowerings__
    assert kernels.mfma_gfx950.__hc_has_fallback__
    # Lane layout of the 32x32x16 accumulator: every (row, col) once.
    seen = {(r, kernels.lane_column(l)) for l in range(64) for r in kernels.lane_acc_rows(l)}
    assert seen == {(r, c) for r in range(32) for c in range(32)}


def test_symbols_interned_eval_and_conflicts():
    assert sym.M is sym.M
    e = ceil_div(sym.M, 16) * 32
    assert e.eval({sym.M: 17}) == 64 and e.eval({"M": 32}) == 64
    b = Bindings()
    b.bind(sym.K, 7, source="a.shape[1]")
    b.bind(sym.K, 7, source="b.shape[0]")
    with pytest.raises(SymbolConflictError, match="conflicting binding for K: 7 from 'b.shape\\[0\\]' vs 8"):
        b.bind(sym.K, 8, source="b.shape[0]")
    b.require(sym.K * 2, 14)
    with pytest.raises(SymbolConflictError):
        b.require(sym.K + 1, 7, source="x")


def _arrays(m, n, k, dt=np.float16):
    return np.zeros((m, k), dt), np.zeros((k, n), dt), np.zeros((m, n), np.float32)


def test_prepare_launch_geometry_of_the_reference_kernel():
    a, b, c = _arrays(100, 70, 30)
    p = prepare_launch(_kernels.tiled_gfx11_wmma_matmul, (a, b, c), {}, g.Gfx950Target())
    assert p.work_shape == (7 * 32, 5) and p.group_shape == (32, 1) and p.subgroup_size == 32
    assert p.env[sym.M] == 100 and p.env[sym.N] == 70 and p.env[sym.K] == 30
    assert p.buffer_params == ("a", "b", "c")


@pytest.mark.parametrize(
    "args,match",
    [
        (lambda: (np.zeros((4, 5), np.float32), np.zeros((5, 6), np.float16), np.zeros((4, 6), np.float32)),
         "a dtype expected float16, got float32"),
        (lambda: (np.zeros((4, 5), np.float16), np.zeros((6, 6), np.float16), np.zeros((4, 6), np.float32)),
         "conflicting binding for K"),
        (lambda: (np.zeros((4,), np.float16), np.zeros((5, 6), np.float16), np.zeros((4, 6), np.float32)),
         "a rank does not match its Buffer annotation"),
        (lambda: ([[1.0]], np.zeros((1, 6), np.float16), np.zeros((1, 6), np.float32)),
         "a must be a numpy.ndarray or torch.Tensor buffer"),
    ],
)
def test_launch_errors_before_execution(args, match):
    with pytest.raises(LaunchError, match=match):
        g.launch(_kernels.tiled_gfx11_wmma_matmul, *args(), target=g.Gfx950Target())


def test_launch_requires_a_kernel_and_a_lowering():
    with pytest.raises(LaunchError, match="decorated with @kernel"):
        g.launch(lambda group: None)
    a, b, c = _arrays(4, 4, 4)
    with pytest.raises(LaunchError, match="no amdgpu-gfx950 lowering for kernel 'some_other_kernel'"):
        g.launch(_kernels.some_other_kernel, a, b, c)
    with pytest.raises(LaunchError, match="no amdgpu-gfx950 lowering"):
        g.launch(_kernels.tiled_gfx950_mfma_matmul, np.zeros((4,), np.float16))


def test_the_reference_kernel_is_recognised_as_the_contraction():
    from hc.gfx950 import _contract

    got = _contract.recognise(_kernels.tiled_gfx11_wmma_matmul)
    assert got.tile == (16, 16, 16) and got.dtype == "float16" and (got.a, got.b, got.c) == ("a", "b", "c")
    assert got.intrinsics == ("wmma_gfx11",)
    assert g.find_lowering(_kernels.tiled_gfx11_wmma_matmul).contraction == got


def test_the_package_kernels_are_recognised_through_their_mfma_intrinsic():
    from hc.gfx950 import _contract, kernels

    for fn, dtype in ((kernels.tiled_gfx950_mfma_matmul, "float16"),
                      (kernels.tiled_gfx950_mfma_matmul_bf16, "bfloat16")):
        got = _contract.recognise(fn)
        assert got.tile == (32, 32, 16) and got.dtype == dtype and got.intrinsics == ("mfma_gfx950",)
        assert got.ops == ("rocdl.mfma.f32.32x32x16",)
    for fn, dtype in ((kernels.tiled_gfx950_mfma16_matmul, "float16"),
                      (kernels.tiled_gfx950_mfma16_matmul_bf16, "bfloat16")):
        got = _contract.recognise(fn)
        assert got.tile == (16, 16, 32) and got.dtype == dtype and got.intrinsics == ("mfma16_gfx950",)
        assert got.ops == ("rocdl.mfma.f32.16x16x32",)
    assert _contract.recognise(_kernels.tiled_gfx11_wmma_matmul).ops == ("amdgpu.wmma",)


def _wave_inputs(m, n, k, seed, dtype="float16", ints=False):
    rng = np.random.default_rng(seed)
    if ints:
        a = rng.integers(-8, 9, (m, k)).astype(np.float32)
        b = rng.integers(-8, 9, (k, n)).astype(np.float32)
    else:
        a = rng.normal(0, 1, (m, k)).astype(np.float32)
        b = rng.normal(0, 1, (k, n)).astype(np.float32)
    if dtype == "float16":
        a, b = a.astype(np.float16), b.astype(np.float16)
    else:
        from hc.gfx950.workloads import f32_to_bf16_bits

        a, b = f32_to_bf16_bits(a), f32_to_bf16_bits(b)
    return a, b, rng.random((m, k)) < 0.8, rng.random((k, n)) < 0.8


def test_fallback_wave_of_both_intrinsics_is_one_masked_matrix_step():
    """fallback_wave runs the fallback body per lane; placed by the stated
    lane layout the 64 results are acc + A @ B of the masked operands, as the
    oracle's sequential float32 fold (every intrinsic, both dtypes)."""
    import hc_oracle as oracle
    from hc.gfx950 import intrinsics, kernels

    cases = ((kernels.mfma_gfx950, 32, 16, kernels.lane_acc_rows, kernels.lane_column),
             (kernels.mfma16_gfx950, 16, 32, kernels.lane16_acc_rows, kernels.lane16_column))
    for fn, mn, k, rows_of, col_of in cases:
        for dtype in ("float16", "bfloat16"):
            a, b, am, bm = _wave_inputs(mn, mn, k, 5, dtype)
            code = oracle.F16 if dtype == "float16" else oracle.BF16
            a0 = np.where(am, a, np.zeros_like(a))
            b0 = np.where(bm, b, np.zeros_like(b))
            regs = mn * mn // 64
            got = intrinsics.fallback_wave(fn, a, b, np.zeros((64, regs), np.float32), dtype=dtype, a_mask=am,
                                           b_mask=bm, wave_size=64, arch="gfx950")
            c = np.full((mn, mn), np.nan, np.float32)
            for lane in range(64):
                for r, row in enumerate(rows_of(lane)):
                    c[row, col_of(lane)] = got[lane, r]
            assert np.array_equal(c, oracle.gemm_sequential(a0, b0, code)), (fn.__name__, dtype)


def test_lowering_is_called_through_a_recording_ctx():
    from hc.gfx950 import intrinsics, kernels

    for fn, shape in ((kernels.mfma_gfx950, (32, 32, 16)), (kernels.mfma16_gfx950, (16, 16, 32))):
        m, n, k = shape
        a, b, _, _ = _wave_inputs(m, n, k, 1)
        name, got = intrinsics.lowered_op(fn, a, b, np.zeros((64, m * n // 64), np.float32), wave_size=64,
                                          arch="gfx950")
        assert got == shape and name == f"rocdl.mfma.f32.{m}x{n}x{k}"
    # another instruction, declared by an intrinsic's lowering: refused before any device call
    a, b, _, _ = _wave_inputs(32, 32, 16, 1)
    with pytest.raises(LaunchError, match=r"creates 'rocdl.mfma.f32.32x32x8', which no kernel of this library"):
        intrinsics.run_wave(_kernels.mfma_k8_gfx950, a, b, np.zeros((64, 16), np.float32), wave_size=64,
                            arch="gfx950")


def test_lowerings_that_misstate_the_op_are_refused():
    from hc.core import vector_type
    from hc.gfx950 import _lowering, kernels

    args = ("group", "a", "b", "acc")

    def intrinsic_with(lower):
        @kernel.intrinsic(scope=WorkItem, effects="pure", const_attrs={"wave_size", "arch"},
                          result_types=(vector_type((16,), np.float32),))
        def probe_mfma(group, a_tile, b_tile, acc_frag, *, lane, wave_size, arch):
            return acc_frag

        probe_mfma.lower(target="amdgpu-gfx950")(lower)
        return probe_mfma

    def op(ctx, name="rocdl.mfma.f32.32x32x16", results=None, operands=None, **attrs):
        full = {"arch": "gfx950", "wave_size": 64, "m": 32, "n": 32, "k": 16, **attrs}
        return ctx.builder.create(name, results=results if results is not None else [ctx.result_type(0)],
                                  operands=operands if operands is not None else ["a", "b", "acc"], attrs=full,
                                  loc=ctx.loc)

    def check(lower, match):
        fn = intrinsic_with(lower)
        with pytest.raises(_lowering.LoweringError, match=match):
            recorded = _lowering.record_lowering(fn, "amdgpu-gfx950", args, {"lane": 0, "wave_size": 64,
                                                                            "arch": "gfx950"})
            _lowering.check_matrix_op(recorded, "amdgpu-gfx950", fn, args)

    check(lambda ctx, *a, **k: op(ctx, k=8).result(0), r"declares k=8, but that instruction has k=16")
    check(lambda ctx, *a, **k: op(ctx, arch="gfx942").result(0), r"declares arch='gfx942'")
    check(lambda ctx, *a, **k: op(ctx, wave_size=32).result(0), r"declares wave_size=32")
    check(lambda ctx, *a, **k: op(ctx, name="rocdl.mfma.f32.16x16x32", m=16, n=16, k=32).result(0),
          r"results are .*not one VectorTypeSpec\(dimensions=\(4,\)")
    check(lambda ctx, *a, **k: op(ctx, operands=["acc", "b", "a"]).result(0), "accumulator")
    check(lambda ctx, *a, **k: (op(ctx), op(ctx))[0].result(0), "creates 2 ops")
    check(lambda ctx, *a, **k: op(ctx) and None, "does not return result 0")
    check(lambda ctx, *a, **k: ctx.builder.create("rocdl.mfma.f32.32x32x16", results=[ctx.result_type(1)]),
          "declares 1 result types")
    assert _lowering.lowering_target(kernels.mfma_gfx950) == "amdgpu-gfx950"
    assert _lowering.lowering_target(_kernels.wmma_gfx11) == "amdgpu-gfx11"


@pytest.mark.parametrize(
    "name,reason",
    [
        ("transposed_store_kernel", r"probe computes \d+ elements of c that differ from A @ B"),
        ("k_step_32_kernel", r"K step \(32\) must equal the tiles' K extent"),
        ("no_accumulate_kernel", "two tile loads and one accumulate"),
        ("short_k_kernel", r"K loop must run to a.shape\[1\]"),
        ("half_grid_kernel", r"leaves \d+ elements of c unwritten"),
        ("unlowered_kernel", "has no lowering registered for an amdgpu target"),
        ("some_other_kernel", "the body must be"),
        ("f16_fold_kernel", r"probe with partial sums that need float32 accumulation computes \d+ elements"),
        ("clamped_kernel", r"probe with partial sums that need float32 accumulation computes \d+ elements"),
        ("f16_result_kernel", "helper 'f16_result_step' returns a float16 accumulator, not float32"),
        ("wrong_shape_kernel", r"creates 'rocdl.mfma.f32.32x32x8', which no kernel of this library executes"),
    ],
)
def test_near_misses_are_rejected_with_the_reason(name, reason):
    fn = getattr(_kernels, name)
    a, b, c = _arrays(4, 4, 4)
    with pytest.raises(LaunchError, match=rf"no amdgpu-gfx950 lowering for kernel '{name}': .*{reason}"):
        g.launch(fn, a, b, c, target=g.Gfx950Target())
    with pytest.raises(LaunchError, match=reason):
        hc.compile(fn)


def test_a_kernel_with_the_reference_name_and_another_body_is_rejected():
    from . import _kernels_same_name

    fn = _kernels_same_name.tiled_gfx11_wmma_matmul
    assert fn.__name__ == _kernels.tiled_gfx11_wmma_matmul.__name__
    with pytest.raises(LaunchError, match="differ from A @ B"):
        g.find_lowering(fn)
    with pytest.raises(LaunchError, match="differ from A @ B"):
        g.register_kernel(fn)


def test_register_kernel_checks_the_body_or_takes_a_callable():
    assert g.register_kernel(_kernels.tiled_gfx11_wmma_matmul) is _kernels.tiled_gfx11_wmma_matmul
    with pytest.raises(LaunchError, match="the body must be"):
        g.register_kernel(_kernels.some_other_kernel)
    seen = []
    g.register_kernel(_kernels.some_other_kernel, lambda prepared, target: seen.append(prepared.env))
    try:
        g.launch(_kernels.some_other_kernel, *_arrays(4, 5, 6))
        assert seen and seen[0][sym.N] == 5
    finally:
        g._LOWERINGS.pop(_kernels.some_other_kernel)


def test_a_verify_hook_failure_rejects_the_kernel(monkeypatch):
    from hc.gfx950 import _contract

    def refuse(sig, target):
        raise ValueError("not on this target")

    monkeypatch.setattr(_kernels.wmma_gfx11, "__hc_verify__", refuse)
    _contract.forget(_kernels.tiled_gfx11_wmma_matmul)
    try:
        with pytest.raises(LaunchError, match="verify hook failed: not on this target"):
            g.find_lowering(_kernels.tiled_gfx11_wmma_matmul)
    finally:
        monkeypatch.undo()
        _contract.forget(_kernels.tiled_gfx11_wmma_matmul)
    assert g.find_lowering(_kernels.tiled_gfx11_wmma_matmul).contraction.tile == (16, 16, 16)


def test_zero_size_launch_is_a_noop_on_every_target():
    a, b, c = _arrays(0, 5, 3)
    g.launch(_kernels.tiled_gfx11_wmma_matmul, a, b, c)  # no GPU needed: nothing runs
    hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, a, b, c, target=SimulatorTarget())


def test_simulator_target_validates_then_reports_no_interpreter(monkeypatch):
    monkeypatch.setenv("HC_DEFAULT_TARGET", "simulator")
    a, b, c = _arrays(4, 4, 4)
    with pytest.raises(LaunchError, match="conflicting binding"):
        hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, a, np.zeros((5, 4), np.float16), c)
    with pytest.raises(SimulatorError, match="host simulator is not part of this build"):
        hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, a, b, c)
    with pytest.raises(SimulatorError, match="host simulator is not part of this build"):
        hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, a, b, c, target=SimulatorTarget())
    with pytest.raises(LaunchError, match="group size exceeds"):
        hc.simulator.launch(_kernels.tiled_gfx11_wmma_matmul, a, b, c, target=SimulatorTarget(max_group_size=16))


def test_default_target_switch(monkeypatch):
    monkeypatch.setenv("HC_DEFAULT_TARGET", "gfx950")
    assert isinstance(hc.simulator.default_target(), g.Gfx950Target)
    monkeypatch.setenv("HC_DEFAULT_TARGET", "simulator")
    assert isinstance(hc.simulator.default_target(), SimulatorTarget)
    # Unset: gfx950 exactly when a gfx950 device and the library are there.
    monkeypatch.delenv("HC_DEFAULT_TARGET")
    monkeypatch.setattr(g, "device_available", lambda: True)
    assert isinstance(hc.simulator.default_target(), g.Gfx950Target)
    monkeypatch.setattr(g, "device_available", lambda: False)
    assert isinstance(hc.simulator.default_target(), SimulatorTarget)


def test_compile_handle_checks_lowering_and_pinned_symbols():
    handle = hc.compile(_kernels.tiled_gfx11_wmma_matmul, symbols={"K": 8})
    assert isinstance(handle, hc.CompiledKernel)
    a, b, c = _arrays(4, 4, 7)
    with pytest.raises(LaunchError, match="K is compiled as 8 but the arguments bind 7"):
        handle(a, b, c)
    with pytest.raises(LaunchError, match="no amdgpu-gfx950 lowering"):
        hc.compile(_kernels.some_other_kernel)


def test_gemm_entry_validates_before_touching_a_device():
    pytest.importorskip("torch")
    with pytest.raises(LaunchError, match="A.shape\\[1\\] must match B.shape\\[0\\]"):
        g.gemm(np.zeros((2, 3), np.float16), np.zeros((4, 2), np.float16))
    with pytest.raises(LaunchError, match="must both be float16 or both bfloat16"):
        g.gemm(np.zeros((2, 3), np.float16), np.zeros((3, 2), np.float32))
    with pytest.raises(LaunchError, match="unknown algo"):
        g.gemm(np.zeros((2, 3), np.float16), np.zeros((3, 2), np.float16), algo="fast")
    with pytest.raises(LaunchError, match="C shape"):
        g.gemm(np.zeros((2, 3), np.float16), np.zeros((3, 2), np.float16), out=np.zeros((3, 3), np.float32))


def test_gfx950_intrinsic_fallback_body_is_one_mfma_step():
    """Run the wave64 intrinsic's fallback body for all 64 lanes (stand-in
    tile and group objects) and assemble the 32x32 result from the stated
    lane layout: it must equal acc + A @ B as the oracle's sequential float32
    fold, with masked-off (inactive) operand entries counting as +0."""
    import hc_oracle as oracle
    from hc.gfx950 import kernels

    class Tile:
        def __init__(self, data, active):
            self.data, self.active = data, active

        def with_inactive(self, value):
            return np.where(self.active, self.data, np.asarray(value, dtype=self.data.dtype))

    class Group:
        @staticmethod
        def vload(values, shape):
            assert tuple(shape) == (kernels.ACC_REGS,)
            return np.asarray(values, dtype=np.float32)

    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, (32, 16)).astype(np.float16)
    b = rng.uniform(-1, 1, (16, 32)).astype(np.float16)
    a_act = rng.random(a.shape) < 0.9
    b_act = rng.random(b.shape) < 0.9
    a0 = np.where(a_act, a, np.float16(0))
    b0 = np.where(b_act, b, np.float16(0))

    def run(acc0):
        out = np.full((32, 32), np.nan, dtype=np.float32)
        for lane in range(64):
            rows = kernels.lane_acc_rows(lane)
            col = kernels.lane_column(lane)
            frag = np.array([acc0[r, col] for r in rows], dtype=np.float32)
            res = kernels.mfma_gfx950(Group, Tile(a, a_act), Tile(b, b_act), frag, lane=lane, wave_size=64,
                                      arch="gfx950")
            for reg, r in enumerate(rows):
                out[r, col] = res[reg]
        return out

    # From zero accumulators: exactly the oracle's fold of the masked operands.
    assert np.array_equal(run(np.zeros((32, 32), np.float32)), oracle.gemm_sequential(a0, b0))
    # From nonzero accumulators: the fold continues from them, k ascending.
    acc0 = rng.uniform(-4, 4, (32, 32)).astype(np.float32)
    want = acc0.copy()
    for k in range(16):
        want = (want + a0[:, k : k + 1].astype(np.float32) * b0[k : k + 1, :].astype(np.float32)).astype(np.float32)
    assert np.array_equal(run(acc0), want)
