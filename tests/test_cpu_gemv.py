"""The fp16 GEMV of HELM's CPU stages (helm/kernels): libhelm_cpu.so against
the float64 oracle (oracle/gemv.py), HELM's own test cases
(tests/unit/runtime/test_kernels.py), the module-patching surface, and the
oracle pinned by exact integer cases and torch's float32 F.linear."""
import os
import re

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from helm_amd import kernels
from oracle import gemv as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "helm_cpu.h")

needs_kernel = pytest.mark.skipif(not kernels.is_available(),
                                  reason=f"native GEMV unavailable: {kernels.load_error()}")


# Every test here runs twice: in the CPU suite, and under the `gpu` marker so
# that the GPU run exercises the host-CPU code on the host CPU of the machine
# that holds the GPU (another microarchitecture than the build machine's).
@pytest.fixture(autouse=True, params=[pytest.param("host", id="host"),
                                      pytest.param("gpu_host", id="gpu_host", marks=pytest.mark.gpu)])
def _where(request):
    return request.param


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(*shape, generator=g)).half()


def _check(y, x, W, b=None):
    yv = y.reshape(-1).double().numpy()
    ex = O.gemv_fp64(x.reshape(-1).numpy(), W.numpy(), None if b is None else b.numpy())
    bound = O.error_bound(x.reshape(-1).numpy(), W.numpy(), None if b is None else b.numpy())
    err = np.abs(yv - ex)
    assert (err <= bound).all(), f"max excess {(err - bound).max()}"


# ---- the oracle, pinned ------------------------------------------------------

def test_oracle_exact_on_small_integers():
    """Integer W, x (|v| <= 8) and bias: every product and partial sum is an
    integer below 2^11, exact in fp16, fp32 and fp64 — the oracle's value is
    the integer dot product by brute force."""
    rng = np.random.default_rng(3)
    W = rng.integers(-3, 4, size=(7, 11)).astype(np.float16)
    x = rng.integers(-8, 9, size=11).astype(np.float16)
    b = rng.integers(-5, 6, size=7).astype(np.float16)
    brute = [sum(int(W[i, j]) * int(x[j]) for j in range(11)) + int(b[i]) for i in range(7)]
    assert O.fp16_linear_ref(x, W, b).astype(np.int64).tolist() == brute


def test_oracle_closed_forms_and_torch():
    """Identity W returns x; a one-hot x returns W's column; random inputs
    agree with torch's float32 F.linear within the float32 bound."""
    x = _rand((33,), 1).numpy()
    assert np.array_equal(O.fp16_linear_ref(x, np.eye(33, dtype=np.float16)), x)
    W = _rand((9, 33), 2).numpy()
    e = np.zeros(33, dtype=np.float16)
    e[5] = 1.0
    assert np.array_equal(O.fp16_linear_ref(e, W), W[:, 5])
    xt, Wt = _rand((257,), 4), _rand((40, 257), 5)
    t = F.linear(xt.float(), Wt.float()).double().numpy()
    ex = O.gemv_fp64(xt.numpy(), Wt.numpy())
    assert (np.abs(t - ex) <= O.error_bound(xt.numpy(), Wt.numpy())).all()
    # the bound is not vacuous: dropping a term breaks it
    wrong = ex - Wt.numpy()[:, -1].astype(np.float64) * xt.numpy()[-1]
    assert (np.abs(wrong - ex) > O.error_bound(xt.numpy(), Wt.numpy())).any()


# ---- the C-ABI -----------------------------------------------------------------

def test_library_exports_the_header():
    assert kernels.LIB_PATH.exists(), "run python -m helm_amd.build"
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    declared = set(re.findall(r"\b(helm_cpu_[a-z_0-9]+)\s*\(", src))
    syms = os.popen(f"nm -D --defined-only {kernels.LIB_PATH}").read()
    assert set(re.findall(r" T (helm_[a-z_0-9]+)", syms)) == declared


@needs_kernel
def test_argument_errors():
    with pytest.raises(ValueError):
        kernels.gemv_fp16(_rand((8,), 0), _rand((4, 9), 1))
    with pytest.raises(ValueError):
        kernels.gemv_fp16(_rand((8,), 0), _rand((4, 8), 1).float())
    with pytest.raises(ValueError):
        kernels.gemv_fp16(_rand((8,), 0), _rand((4, 8), 1), bias=_rand((5,), 2))


# ---- parity ----------------------------------------------------------------------

@needs_kernel
@pytest.mark.parametrize("isa", ["auto", "avx2"])
@pytest.mark.parametrize("N,K,bias", [(512, 256, None), (64, 128, "fp16"), (77, 131, None),
                                      (1, 1, "fp32"), (3, 17, "fp16"), (130, 4099, "fp32"),
                                      (4096, 4096, None)])
def test_gemv_matches_oracle(N, K, bias, isa, monkeypatch):
    """Shapes from HELM's tests (512x256, 64x128 with bias, 77x131 odd tails)
    plus row counts that are not multiples of 4, K below one vector, a
    Qwen3-8B projection (4096x4096), fp16 and fp32 biases; AVX-512 and AVX2
    paths (the library reads HELM_CPU_ISA per call)."""
    if isa == "avx2":
        monkeypatch.setenv("HELM_CPU_ISA", "avx2")
    x, W = _rand((K,), 10 + N), _rand((N, K), 20 + K)
    b = None
    if bias == "fp16":
        b = _rand((N,), 30)
    elif bias == "fp32":
        b = torch.randn(N, generator=torch.Generator().manual_seed(31))
    y = kernels.gemv_fp16(x, W, b)
    assert y.dtype == torch.float16 and y.shape == (N,)
    _check(y, x, W, b)


@needs_kernel
def test_threads_do_not_change_the_result():
    """Rows are independent: any thread count gives bit-identical output."""
    x, W = _rand((1000,), 40), _rand((333, 1000), 41)
    ys = [kernels.gemv_fp16(x, W, threads=t) for t in (1, 2, 3, 8, 0)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


@needs_kernel
def test_overflow_and_special_values_round_like_torch():
    """Sums past fp16's range become inf, as torch's float32 -> fp16 cast does;
    a NaN weight gives NaN in its row only."""
    K = 64
    x = torch.full((K,), 60.0).half()
    W = torch.full((3, K), 30.0).half()          # 64 * 1800 = 115200 > 65504
    W[1] = -30.0
    W[2] = 0.0
    W[2, 7] = float("nan")
    y = kernels.gemv_fp16(x, W)
    assert y[0].item() == float("inf") and y[1].item() == float("-inf")
    assert torch.isnan(y[2])
    ref = F.linear(x.float(), W.float()).half()
    assert torch.equal(y[:2], ref[:2])


# ---- HELM's module surface (tests/unit/runtime/test_kernels.py) -----------------------

def _ref(x, w, b=None):
    return F.linear(x.float(), w.float(), b.float() if b is not None else None).half()


@needs_kernel
def test_fp16_linear_decode_path():
    torch.manual_seed(0)
    x = torch.randn(1, 1, 256, dtype=torch.float16)
    w = torch.randn(512, 256, dtype=torch.float16)
    out = kernels.fp16_linear(x, w)
    assert out.dtype == torch.float16 and out.shape == (1, 1, 512)
    assert torch.allclose(out.float(), _ref(x, w).float(), atol=2e-2, rtol=1e-2)
    _check(out, x, w)


@needs_kernel
def test_fp16_linear_with_bias():
    torch.manual_seed(1)
    x = torch.randn(1, 1, 128, dtype=torch.float16)
    w = torch.randn(64, 128, dtype=torch.float16)
    b = torch.randn(64, dtype=torch.float16)
    out = kernels.fp16_linear(x, w, b)
    assert torch.allclose(out.float(), _ref(x, w, b).float(), atol=2e-2, rtol=1e-2)
    _check(out, x, w, b)


def test_fp16_linear_prefill_and_passthrough():
    """More than one token: HELM's float32 GEMM branch, exactly; fp32 inputs:
    plain F.linear, exactly (these run with or without the native library)."""
    torch.manual_seed(3)
    x = torch.randn(2, 5, 64, dtype=torch.float16)
    w = torch.randn(32, 64, dtype=torch.float16)
    b = torch.randn(32, dtype=torch.float16)
    assert torch.equal(kernels.fp16_linear(x, w, b), _ref(x, w, b))
    xf, wf = x.float(), w.float()
    assert torch.equal(kernels.fp16_linear(xf, wf), F.linear(xf, wf))


@needs_kernel
def test_disable_env_takes_the_float32_branch(monkeypatch):
    monkeypatch.setenv("HELM_DISABLE_AVX", "1")
    x = _rand((1, 1, 96), 50)
    w = _rand((48, 96), 51)
    assert torch.equal(kernels.fp16_linear(x, w), _ref(x, w))


@needs_kernel
def test_patch_cpu_linears():
    """Every fp16 CPU nn.Linear (nested too) is routed through the native
    GEMV in place — same module objects and parameters; fp32 linears are left
    alone; decode outputs follow the GEMV; a second call routes nothing new."""
    torch.manual_seed(4)
    m = nn.Sequential(nn.Linear(64, 32), nn.ReLU(),
                      nn.Sequential(nn.Linear(32, 16), nn.Linear(16, 8).float()))
    m[0].half()
    m[2][0].half()
    lin0, w0 = m[0], m[0].weight
    keys = list(m.state_dict())
    assert kernels.patch_cpu_linears(m) == 2
    assert m[0] is lin0 and isinstance(m[0], nn.Linear) and m[0].weight is w0
    assert type(m[0]) is kernels.NativeLinear and type(m[2][1]) is nn.Linear
    assert list(m.state_dict()) == keys
    assert kernels.patch_cpu_linears(m) == 0
    # HELM walks the children only: a bare linear passed in is not patched
    bare = nn.Linear(8, 4).half()
    assert kernels.patch_cpu_linears(bare) == 0 and type(bare) is nn.Linear
    x = torch.randn(1, 1, 64, dtype=torch.float16)
    y = m[0](x)
    assert torch.equal(y.reshape(-1), kernels.gemv_fp16(x, m[0].weight, m[0].bias).reshape(-1))
    # the fp32 linear still runs F.linear; a prefill-sized input takes HELM's fp32 branch
    xf = torch.randn(3, 16)
    assert torch.equal(m[2][1](xf), F.linear(xf, m[2][1].weight, m[2][1].bias))
    xp = torch.randn(2, 9, 64, dtype=torch.float16)
    assert torch.equal(m[0](xp), F.linear(xp.float(), w0.float(), m[0].bias.float()).half())


@needs_kernel
def test_patched_model_saves_and_loads(tmp_path):
    """A patched model goes through torch.save / torch.load (whole module and
    state_dict) and gives the same decode outputs afterwards."""
    torch.manual_seed(6)
    m = nn.Sequential(nn.Linear(64, 32), nn.ReLU(), nn.Linear(32, 16)).half()
    assert kernels.patch_cpu_linears(m) == 2
    x = torch.randn(1, 64, dtype=torch.float16)
    y = m(x)
    torch.save(m, tmp_path / "m.pt")
    torch.save(m.state_dict(), tmp_path / "sd.pt")
    m2 = torch.load(tmp_path / "m.pt", weights_only=False)
    assert type(m2[0]) is kernels.NativeLinear
    assert torch.equal(m2(x), y)
    m3 = nn.Sequential(nn.Linear(64, 32), nn.ReLU(), nn.Linear(32, 16)).half()
    m3.load_state_dict(torch.load(tmp_path / "sd.pt", weights_only=True))
    assert kernels.patch_cpu_linears(m3) == 2
    assert torch.equal(m3(x), y)


def test_fp16_linear_empty_input_takes_the_float32_branch():
    """Zero tokens: F.linear's empty [..., N] result, as HELM gives it."""
    w = torch.randn(8, 16).half()
    y = kernels.fp16_linear(torch.zeros(0, 16, dtype=torch.float16), w)
    assert y.shape == (0, 8) and y.dtype == torch.float16


# ---- against HELM's own kernel, built from its source by oracle/build_ref.py ------------

def _ref_module():
    from oracle import build_ref
    return build_ref.load()


@pytest.mark.parametrize("N,K,bias", [(512, 256, False), (64, 128, True), (77, 131, False),
                                      (1000, 3000, True)])
def test_reference_kernel_within_oracle_bound_and_beside_ours(N, K, bias):
    """HELM's helm_fp16_linear (its AVX2 GEMV) lies within the oracle's bound
    — which pins the oracle to the reference's arithmetic — and the native
    GEMV here differs from it by at most one fp16 ulp (both round one float32
    sum, accumulated in different orders)."""
    mod = _ref_module()
    if mod is None:
        pytest.skip("oracle/_ref not built (the reference tree is absent)")
    x, W = _rand((1, 1, K), 60 + N), _rand((N, K), 61 + K)
    b = _rand((N,), 62) if bias else None
    yr = mod.helm_fp16_linear(x, W, b)
    assert yr.shape == (1, 1, N) and yr.dtype == torch.float16
    _check(yr, x, W, b)
    if kernels.is_available():
        y = kernels.fp16_linear(x, W, b)
        d = (y.float() - yr.float()).abs()
        ulp = torch.finfo(torch.float16).eps * yr.float().abs().clamp_min(2.0 ** -14)
        assert (d <= ulp).all()


# ---- up to 8 tokens per call (a batched decode step) ------------------------------------

@needs_kernel
@pytest.mark.parametrize("isa", ["auto", "avx2"])
@pytest.mark.parametrize("M", [2, 3, 4, 5, 7, 8])
def test_batch_is_invariant_and_within_oracle(M, isa, monkeypatch):
    """M vectors in one call (W read once): each output row equals that
    vector's row in a two-vector call bit for bit (the batched kernel's
    summation order depends on K alone, not on the batch size, grouping or
    thread count), and lies within the oracle's bound, as the one-vector call
    (its own order) does; odd N and K exercise every tail."""
    if isa == "avx2":
        monkeypatch.setenv("HELM_CPU_ISA", "avx2")
    N, K = 203, 517
    x, W, b = _rand((M, K), 70 + M), _rand((N, K), 71), _rand((N,), 72)
    y = kernels.gemv_fp16(x, W, b)
    assert y.shape == (M, N)
    assert torch.equal(kernels.gemv_fp16(x, W, b, threads=3), y)
    for m in range(M):
        pair = torch.stack([x[m], x[(m + 1) % M]])
        assert torch.equal(y[m], kernels.gemv_fp16(pair, W, b)[0])
        _check(y[m], x[m], W, b)
        _check(kernels.gemv_fp16(x[m], W, b), x[m], W, b)


@needs_kernel
def test_fp16_linear_small_batches_native_larger_fp32():
    """2..8 tokens (any leading shape) take the native GEMV, within the
    oracle's bound of HELM's float32 branch; 9 tokens take HELM's float32
    branch exactly."""
    w, b = _rand((96, 160), 80), _rand((96,), 81)
    for shape in [(2, 1, 160), (1, 8, 160), (2, 2, 2, 160)]:
        x = _rand(shape, 82)
        out = kernels.fp16_linear(x, w, b)
        assert out.shape == shape[:-1] + (96,)
        flat = x.reshape(-1, 160)
        for m in range(flat.shape[0]):
            _check(out.reshape(-1, 96)[m], flat[m], w, b)
        assert torch.allclose(out.float(), _ref(x, w, b).float(), atol=2e-2, rtol=1e-2)
    x9 = _rand((9, 160), 83)
    assert torch.equal(kernels.fp16_linear(x9, w, b), _ref(x9, w, b))
    with pytest.raises(ValueError):
        kernels.gemv_fp16(x9, w)
