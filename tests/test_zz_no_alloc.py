"""The launch that allocates nothing (lunaflux_hip_function_launch_scratch)
against the existing launch (lunaflux_hip_function_launch) on the same
kernels, through the C ABI.

The split-K W8A16 entries take their workspace (fp32 partial tiles and
arrival counters, which must start at zero) as the last kernel argument. The
existing path passes a caller allocation, zero-filled once; the scratch path
passes the library's per-device scratch array, cleared by the library before
the launch. Two calls in a row share that array, the second with fewer live
rows and a smaller workspace whose counters sit where the first call's
partial tiles were: both must be bit-identical to the existing entry point.
"""
import numpy as np
import pytest

from lunaflux_amd import _abi, synth
from lunaflux_amd.device import DeviceError, KernelArguments
from lunaflux_amd.fp8 import _region

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    from lunaflux_amd.fp8 import ProjectionRuntime
    return ProjectionRuntime(0)


def bound_qkv(rt, rng, m, max_tokens):
    k = 4096
    ws = [rt.upload_weight(*synth.weight(rng, n, k)) for n in (4096, 1024, 1024)]
    x = np.concatenate([synth.activations(rng, m, k), np.zeros((max_tokens - m, k), np.uint16)])
    xa, ya = rt.context.upload(x), rt.context.allocate(max_tokens * 6144 * 2)
    op = rt.bind_qkv("w8a16", rt.step_counts(m), _region(xa, alignment=256), *ws,
                     _region(ya, alignment=256), max_tokens)
    return op, ya, (max_tokens, 6144), ws


def bound_down(rt, rng, m, max_tokens):
    k = 14336
    w = rt.upload_weight(*synth.weight(rng, 4096, k))
    x = np.concatenate([synth.activations(rng, m, k), np.zeros((max_tokens - m, k), np.uint16)])
    xa, ya = rt.context.upload(x), rt.context.allocate(max_tokens * 4096 * 2)
    op = rt.bind_dense("w8a16", rt.step_counts(m), _region(xa, alignment=256), w,
                       _region(ya, alignment=256), max_tokens)
    return op, ya, (max_tokens, 4096), [w]


def run_both(rt, op, ya, shape):
    """(output of the existing launch with its allocated workspace, output of
    the scratch launch of the same kernel with the workspace argument left
    to the library)."""
    (step,) = op.steps
    ya.copy_from_host(np.zeros(shape, np.uint16))
    step.function.launch_synchronous(step.dims, step.args, rt.stream)
    ref = ya.read(np.uint16, shape)
    ya.copy_from_host(np.zeros(shape, np.uint16))
    workspace = step.args.arguments[-1]
    regions = KernelArguments(step.args.arguments[:-1])
    step.function.launch_scratch(step.dims, regions, rt.stream, workspace.byte_count, clear=True)
    return ref, ya.read(np.uint16, shape), workspace.byte_count


def test_scratch_launch_matches_the_allocated_workspace_twice(rt):
    rng = np.random.default_rng(7070)
    first = bound_qkv(rt, rng, 32, 32)
    second = bound_down(rt, rng, 7, 32)
    assert first[0].steps[0].name == "lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m32"
    assert second[0].steps[0].name == "lf_fp8_w8a16_dense_k14336_m32"
    ref1, got1, bytes1 = run_both(rt, *first[:3])
    ref2, got2, bytes2 = run_both(rt, *second[:3])
    assert bytes2 < bytes1 <= _abi.LF_SCRATCH_MAX_BYTES
    assert np.any(ref1 != 0) and np.any(ref2[:7] != 0)
    np.testing.assert_array_equal(got1, ref1)
    np.testing.assert_array_equal(got2, ref2)
    assert np.all(got2[7:] == 0)   # rows past the live count stay untouched


def test_scratch_launch_rejects_sizes_and_argument_counts(rt):
    rng = np.random.default_rng(7071)
    op, ya, shape, _ = bound_down(rt, rng, 4, 32)
    (step,) = op.steps
    regions = KernelArguments(step.args.arguments[:-1])
    for size in (0, -1, _abi.LF_SCRATCH_MAX_BYTES + 1):
        with pytest.raises(DeviceError) as err:
            step.function.launch_scratch(step.dims, regions, rt.stream, size)
        assert err.value.status == _abi.LF_INVALID_ARGUMENT
    # 32 regions leave no argument slot for the scratch address
    full = KernelArguments([step.args.arguments[0]] * 32)
    with pytest.raises(DeviceError) as err:
        step.function.launch_scratch(step.dims, full, rt.stream, 256)
    assert err.value.status == _abi.LF_INVALID_ARGUMENT
