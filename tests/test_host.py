"""Host-side checks (no GPU): the C-ABI library exports what the header
declares with the struct layouts the ctypes binding assumes, and the Python
API validates arguments with the reference's exception classes and messages
(compared with texts the reference itself produced, tests/golden/golden.json).
"""

import ctypes
import json
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "namitorch_amd.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nt_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    declared = _declared_functions()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.SIGNATURES), set(declared) ^ set(_native.SIGNATURES)
    assert lib.nt_abi_version() == _native.ABI_VERSION


def test_header_constants_match_python_mirror():
    """Every integer #define of the header that the ctypes layer mirrors has the same value."""
    defines = dict(re.findall(r"^#define (NT_[A-Z0-9_]+) \(?(-?\d+)\)?", HEADER.read_text(), flags=re.M))
    mirrored = {name: value for name, value in defines.items() if hasattr(_native, name)}
    assert {"NT_OK", "NT_F16", "NT_COPY_D2H", "NT_FINALIZE_CLIP_IF_FINITE"} <= set(mirrored)
    for name, value in mirrored.items():
        assert getattr(_native, name) == int(value), name


def test_status_codes_map_to_reference_exceptions():
    lib = _native.load()
    with pytest.raises(ValueError, match="plan output pointer is NULL"):
        _native.check(lib.nt_plan_create(0, None, 0, None, 0, None, None))
    layout = _native.MtLayout(99, 0, 0, -1)
    out = ctypes.c_void_p()
    with pytest.raises(TypeError, match="unsupported dtype"):
        _native.check(lib.nt_plan_create(0, None, 0, ctypes.byref(layout), 0, None, ctypes.byref(out)))
    layout = _native.MtLayout(0, 0, 0, -1)
    with pytest.raises(ValueError, match="multiple of 2048"):
        _native.check(lib.nt_plan_create(0, None, 0, ctypes.byref(layout), 1000, None, ctypes.byref(out)))
    with pytest.raises(ValueError, match="1..16 coefficient slots"):
        _native.check(lib.nt_adamw_mt(ctypes.c_void_p(1), None, 0, None, None))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_struct_layouts_match_header(tmp_path):
    probe = tmp_path / "probe.c"
    probe.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "namitorch_amd.h"\n'
        "int main(void) {\n"
        '  printf("%zu %zu %zu %zu %zu %zu %zu\\n", sizeof(nt_mt_tensor), sizeof(nt_mt_layout), sizeof(nt_adamw_coefs),\n'
        "         sizeof(nt_adamw_coefs64), sizeof(nt_amp_ctrl), sizeof(nt_grad_xform), offsetof(nt_grad_xform, ctrl));\n"
        "  return 0;\n}\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(probe), "-o", str(exe)], check=True)
    sizes = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert sizes == [ctypes.sizeof(_native.MtTensor), ctypes.sizeof(_native.MtLayout), ctypes.sizeof(_native.AdamWCoefs),
                     ctypes.sizeof(_native.AdamWCoefs64), ctypes.sizeof(_native.AmpCtrl), ctypes.sizeof(_native.GradXform),
                     _native.GradXform.ctrl.offset]


@pytest.fixture(scope="module")
def golden_errors(golden_dir):
    return json.loads((golden_dir / "golden.json").read_text())["errors"]


def _param(dtype=np.float32, n=3):
    p = nt.Parameter(np.zeros(n, dtype=dtype))
    p.grad = nt.Tensor(np.zeros(n, dtype=dtype))
    return p


def test_option_errors_match_reference(golden_errors):
    p = _param()
    with pytest.raises(TypeError) as error:
        nt.optim.AdamW([p], fused=1)
    assert str(error.value) == golden_errors["fused_type"]
    with pytest.raises(ValueError) as error:
        nt.optim.AdamW([p], betas=(0.9, 1.0))
    assert str(error.value) == golden_errors["beta_range"]
    with pytest.raises(ValueError) as error:
        nt.optim.clip_grad_norm_([p], -1.0)
    assert str(error.value) == golden_errors["max_norm_negative"]
    with pytest.raises(RuntimeError) as error:
        nt.GradScaler().unscale_(nt.optim.AdamW([p]))
    assert str(error.value) == golden_errors["unscale_before_scale"]


def test_eps_float16_error_matches_reference(golden_errors):
    with pytest.raises(ValueError) as error:
        nt.optim.AdamW([_param(np.float16)], eps=1e-8).step()
    assert str(error.value) == golden_errors["eps_float16"]


def test_fused_true_on_cpu_matches_reference(golden_errors):
    with pytest.raises(RuntimeError) as error:
        nt.optim.AdamW([_param()], fused=True).step()
    assert str(error.value) == golden_errors["fused_true_unsupported"]


def test_cpu_tensors_are_rejected_not_computed():
    p = _param()
    with pytest.raises(RuntimeError, match="only on HIP devices"):
        nt.optim.AdamW([p]).step()
    assert np.array_equal(p.numpy(), np.zeros(3, dtype=np.float32))


def test_gradient_checks_match_reference():
    p = nt.Parameter(np.zeros(3, dtype=np.float32))
    p.grad = nt.Tensor(np.zeros(4, dtype=np.float32))
    with pytest.raises(ValueError, match=r"Gradient shape \(4,\) does not match parameter shape \(3,\)"):
        nt.optim.AdamW([p]).step()
    p.grad = nt.Tensor(np.zeros(3, dtype=np.float64))
    with pytest.raises(TypeError, match="Gradient dtype"):
        nt.optim.AdamW([p]).step()
    with pytest.raises(TypeError, match="bfloat16 parameters require"):
        q = nt.Parameter(np.zeros(3, dtype=np.float32), dtype="bfloat16")
        q.grad = nt.Tensor(np.zeros(3, dtype=np.float32), dtype="bfloat16")
        nt.optim.AdamW([q])._update_many([(q, q.grad, {})])


def test_master_weights_options():
    p = _param()
    with pytest.raises(ValueError, match="state_dtype requires master_weights"):
        nt.optim.AdamW([p], state_dtype="bfloat16")
    with pytest.raises(TypeError, match="state_dtype must be"):
        nt.optim.AdamW([p], master_weights=True, state_dtype="float16")
    opt = nt.optim.AdamW([p], master_weights=True, state_dtype="bfloat16")
    assert "master" in opt._state_buffers


def test_scaler_state_machine_host_only(golden_dir):
    """GradScaler.update arithmetic needs no device: drive it through the
    reference's recorded pattern with the device work stubbed out."""
    record = json.loads((golden_dir / "golden.json").read_text())["scaler"]["scale_sequence"]
    scaler = nt.GradScaler(init_scale=record["init"], growth_factor=record["growth"],
                           backoff_factor=record["backoff"], growth_interval=record["interval"])
    sequence = []
    for overflow in record["pattern"]:
        scaler._optimizer_states = {0: {"stage": "stepped", "finite": not overflow}}
        scaler._scale_used = True
        scaler.update()
        sequence.append(scaler.get_scale())
    assert sequence == record["scale"]
    state = scaler.state_dict()
    assert set(state) == {"version", "scale", "growth_factor", "backoff_factor", "growth_interval", "enabled", "growth_tracker"}
    other = nt.GradScaler()
    other.load_state_dict(state)
    assert other.get_scale() == scaler.get_scale()


def test_state_dict_layout():
    p = _param()
    opt = nt.optim.AdamW([p], lr=3e-4)
    state = opt.state_dict()
    assert state["version"] == 1 and state["param_shapes"] == [[3]]
    assert state["param_groups"][0]["params"] == [0]
    assert state["param_groups"][0]["fused"] is None
    opt.load_state_dict(state)


def test_param_lists_match_survey_counts():
    from namitorch_amd import param_lists as pl
    assert (len(pl.gpt2_shapes()), pl.total_params(pl.gpt2_shapes())) == (148, 124_439_808)
    assert (len(pl.gpt_1p3b_shapes()), pl.total_params(pl.gpt_1p3b_shapes())) == (292, 1_315_819_520)
    assert (len(pl.llama7b_shapes()), pl.total_params(pl.llama7b_shapes())) == (291, 6_738_415_616)


def test_host_bf16_conversion_matches_torch():
    import torch
    rng = np.random.default_rng(2)
    x = rng.standard_normal(10000) * 10
    t = nt.Tensor(x, dtype="bfloat16")
    want = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
    # float64 -> bfloat16 rounds once; torch rounds float32 values, which agree
    # except where the float32 rounding lands on a bfloat16 tie.
    from oracle import lowp
    assert np.array_equal(t.bits(), lowp.f64_to_bf16(x))
    agree = np.mean(t.bits() == want.view(torch.int16).numpy().view(np.uint16))
    assert agree > 0.999


def test_scalar_promotion_matches_reference_fixture_dtypes(golden_dir):
    """The host's promotion and operand rounding (what nt_tensor_scalar is
    given) agree with the reference's result dtypes and with the oracle's
    operand values for every scalar_ops.npz case."""
    from namitorch_amd.dtype import from_numpy_dtype, promote_with_scalar, round_scalar, scalar_dtype
    from oracle import arith
    from test_oracle import scalar_fixture_cases
    data = np.load(golden_dir / "scalar_ops.npz")
    for key, loss, operand, op in scalar_fixture_cases(data):
        tensor_dtype = from_numpy_dtype(loss.dtype)
        kind = scalar_dtype(operand)
        result = promote_with_scalar(tensor_dtype, kind)
        assert result.numpy_dtype == data[key].dtype, key
        want = np.asarray(operand, dtype=arith.operand_dtype(operand)).astype(data[key].dtype)
        assert round_scalar(operand, kind, result) == float(want), key


def test_scalar_promotion_bfloat16_extension():
    from namitorch_amd.dtype import bfloat16, float16, float32, float64, int64, promote_with_scalar, round_scalar
    assert promote_with_scalar(bfloat16, int64) is bfloat16
    assert promote_with_scalar(bfloat16, float16) is float32
    assert promote_with_scalar(bfloat16, float32) is float32
    assert promote_with_scalar(bfloat16, float64) is float64
    assert promote_with_scalar(float16, float32) is float32
    assert round_scalar(3, int64, bfloat16) == 3.0
    assert round_scalar(257, int64, bfloat16) == 256.0        # ties to even at 8 significant bits
    assert round_scalar(259, int64, bfloat16) == 260.0


def test_device_spellings_match_reference(golden_dir):
    """Every Device(value, index) outcome — the device or the exception class
    and message — is the reference's (tests/golden/devices.json)."""
    from namitorch_amd.device import Device
    data = json.loads((golden_dir / "devices.json").read_text())

    def outcome(make):
        try:
            made = make()
            return ["ok", str(made), repr(made)]
        except Exception as error:
            return [type(error).__name__, str(error)]

    for value, index, want in data["spellings"]:
        assert outcome(lambda: Device(value, index)) == want, (value, index)
    for value, index, want in data["copies"]:
        assert outcome(lambda: Device(Device(value), index)) == want, (value, index)
    assert Device("cuda") is Device("cuda:0") is Device("cuda", 0)
    assert Device("cpu") == Device(Device("cpu")) and hash(Device("cuda:2")) == hash(Device("cuda", 2))


def test_host_backend_namespace_is_numpy():
    """backends/__init__.py:79-80: the host backend's namespace is NumPy; the
    HIP namespace offers only constructors and copies (checked on the GPU)."""
    from namitorch_amd import backends
    from namitorch_amd.backends.hip import HIPNamespace
    assert backends.namespace() is np and backends.namespace("cpu") is np
    assert backends.namespace(np.zeros(2, dtype=np.float32)) is np
    assert nt.get_backend("cpu").namespace is np
    probe = HIPNamespace.__new__(HIPNamespace)
    with pytest.raises(RuntimeError, match="'sqrt' is not available"):
        probe.sqrt
    assert not hasattr(probe, "__array_namespace__")


def test_clip_gradient_collection_bulk_path_matches_loop():
    """clip_grad._gradients: the C-level pass for the common case returns what
    the per-parameter loop (clip_grad.py:36-60) returns, and every other case
    (None, repeated, wrong shape, integer) goes through the loop's skips and errors."""
    from namitorch_amd.optim import clip_grad

    def params(n):
        out = []
        for k in range(n):
            p = nt.Parameter(np.zeros(k + 1, dtype=np.float32))
            p.grad = nt.Tensor(np.full(k + 1, k, dtype=np.float32))
            out.append(p)
        return out

    plain = params(5)
    bulk = clip_grad._gradients_bulk(plain)
    assert bulk is not None and all(g is p.grad for g, p in zip(bulk, plain))
    assert [id(g) for g in clip_grad._gradients(tuple(plain))] == [id(g) for g in bulk]
    holes = params(4)
    holes[1].grad = None
    holes[3].grad = holes[2].grad
    assert clip_grad._gradients_bulk(holes) is None
    assert [id(g) for g in clip_grad._gradients(holes)] == [id(holes[0].grad), id(holes[2].grad)]
    wrong = params(3)
    wrong[2].grad = nt.Tensor(np.zeros(7, dtype=np.float32))
    with pytest.raises(ValueError, match=r"Gradient shape \(7,\) does not match parameter shape \(3,\)"):
        clip_grad._gradients(wrong)
    integer = params(2)
    integer[0].grad = nt.Tensor(np.zeros(1, dtype=np.int32))
    with pytest.raises(TypeError, match="Gradients must be floating NamiTorch Tensors."):
        clip_grad._gradients(integer)
    with pytest.raises(TypeError, match="parameters must contain only NamiTorch Tensors."):
        clip_grad._gradients(params(2) + [3])


def test_settled_device_step_never_stalls_the_unsettled_list():
    """A device-decided step that is already settled removes every entry of
    itself from the unsettled list when asked again, so settling the list
    (done by every version read) always ends."""
    from namitorch_amd.amp import DeviceStep
    from namitorch_amd.tensor import _settle_device_steps, _unsettled_steps
    step = DeviceStep.__new__(DeviceStep)           # host state only: no control block, no mirror
    step._reconciled = True
    step.mirror = None
    before = list(_unsettled_steps)
    _unsettled_steps.extend([step, step])
    try:
        _settle_device_steps()
        assert not any(pending is step for pending in _unsettled_steps)
    finally:
        _unsettled_steps[:] = [pending for pending in _unsettled_steps if pending is not step]
    assert _unsettled_steps == before


def test_device_step_rollback_runs_once_across_threads():
    """A skipped device-decided step is rolled back once when two threads
    settle it at the same time (its optimizer's next step on one, a version
    read on another) while its control block is still being waited for: the
    second finds it settled instead of undoing the bookkeeping again."""
    import threading
    import time

    from namitorch_amd.amp import DeviceStep
    from namitorch_amd.tensor import _unsettled_steps

    class SlowStep(DeviceStep):
        def _read_ctrl(self):
            time.sleep(0.05)                # the wait for the finalize (GIL released)
            return self.preset

    gradient = nt.Tensor(np.zeros(4, np.float32))
    gradient._version_counter.value = 7     # the optimistic bump of a clip that did not happen
    step = SlowStep(None, None, unscale=True, honor_skip=True, clip_bumps=[(gradient, 7)])
    step.preset = _native.AmpCtrl()
    step.preset.skip = 1
    step.preset.found_inf = 1
    step.preset.clip = 0
    parameter, first, second = (nt.Tensor(np.zeros(4, np.float32)) for _ in range(3))
    for tensor in (parameter, first, second):
        tensor._version_counter.value = 3   # the optimistic bump of the skipped step included
    state = {"step": 5}
    step.records.append((parameter, state, first, second, None, 5, True, True))
    _unsettled_steps.append(step)
    barrier = threading.Barrier(2)
    errors = []

    def settle():
        try:
            barrier.wait()
            step.reconcile()
        except Exception as error:          # pragma: no cover - reported below
            errors.append(error)

    threads = [threading.Thread(target=settle) for _ in range(2)]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join(10)
    assert not errors
    assert state["step"] == 4
    assert [tensor._version_counter.value for tensor in (parameter, first, second)] == [2, 2, 2]
    assert first._clean_version == 2 and second._clean_version == 2
    assert gradient._version_counter.value == 6
    assert not any(pending is step for pending in _unsettled_steps)


def test_mirror_return_takes_no_lock():
    """Giving a host mirror back takes no lock, so a finalizer that returns
    one while its thread is inside take_mirror (garbage collection can run
    there) cannot deadlock on the pool's lock."""
    from namitorch_amd import runtime
    mirror = _native.AmpMirror()
    address = ctypes.addressof(mirror)
    try:
        with runtime._mirror_lock:
            runtime.give_mirror(mirror, launched=False)
        assert (address, False) in runtime._mirror_returned
    finally:
        # never hand this host-owned struct to a kernel
        runtime._mirror_returned[:] = [entry for entry in runtime._mirror_returned if entry[0] != address]


def test_requires_grad_changes_are_counted():
    """Every change of requires_grad on an existing Tensor moves the count
    that memoized flag checks (the optimizer's step replay) compare."""
    from namitorch_amd.tensor import _requires_grad_changes
    tensor = nt.Tensor(np.zeros(3, np.float32))
    before = _requires_grad_changes.value
    tensor.requires_grad = True
    tensor.requires_grad_(False)
    assert _requires_grad_changes.value == before + 2


def test_writability_is_a_constant():
    """Every Tensor may be written in place and no instance can say
    otherwise: the per-step paths (step replay, GradScaler, clip) rely on
    it instead of scanning the flag."""
    for tensor in (nt.Tensor(np.zeros(3, np.float32)), nt.Parameter(nt.Tensor(np.zeros(3, np.float32)))):
        assert tensor._writable is True
        with pytest.raises(AttributeError):
            tensor._writable = False
        assert tensor._writable is True


def test_registered_cache_sees_a_parameter_moved_between_groups():
    """Moving the last parameter of one group to the front of the next keeps
    the flattened order but changes group membership (and so the options a
    parameter steps with): the registered-parameter cache, whose identity the
    step replay compares, must be rebuilt."""
    params = [nt.Parameter(np.zeros(4, np.float32)) for _ in range(6)]
    optimizer = nt.optim.AdamW([{"params": params[:3], "weight_decay": 0.1}, {"params": params[3:], "weight_decay": 0.0}])
    assert optimizer._registered_parameters() == params
    cache = optimizer.__dict__["_registered_cache"]
    assert optimizer._registered_parameters() == params and optimizer.__dict__["_registered_cache"] is cache
    optimizer.param_groups[1]["params"].insert(0, optimizer.param_groups[0]["params"].pop())
    assert optimizer._registered_parameters() == params
    assert optimizer.__dict__["_registered_cache"] is not cache
    optimizer.param_groups[0]["params"][0] = nt.Parameter(np.zeros(4, np.float32))     # an item replaced in place
    cache = optimizer.__dict__["_registered_cache"]
    assert optimizer._registered_parameters()[0] is optimizer.param_groups[0]["params"][0]
    assert optimizer.__dict__["_registered_cache"] is not cache


def test_runtime_major_version_mismatch_is_refused():
    """The library refuses a HIP runtime of another major version than the
    headers it was built with (PyTorch's bundled runtime could be one), with
    a message naming both and the way out; a newer minor version passes."""
    import ctypes

    from namitorch_amd import _native

    class FakeLibrary:
        def __init__(self, built, runtime):
            self.values = (built, runtime)

        def nt_hip_version(self, built, runtime):
            ctypes.cast(built, ctypes.POINTER(ctypes.c_int32))[0] = self.values[0]
            ctypes.cast(runtime, ctypes.POINTER(ctypes.c_int32))[0] = self.values[1]
            return _native.NT_OK

    saved = _native.HIP_VERSIONS
    try:
        _native._check_runtime(FakeLibrary(70226015, 70051831))        # 7.2 headers, 7.0 runtime
        assert _native.HIP_VERSIONS == (70226015, 70051831)
        with pytest.raises(_native.NativeLibraryError, match=r"built with HIP 7\.2\.26015 but is bound to HIP runtime 6\.4\.0.*NT_SYSTEM_HIP_RUNTIME=1"):
            _native._check_runtime(FakeLibrary(70226015, 60400000))
    finally:
        _native.HIP_VERSIONS = saved
