"""GPU parity of the fp32 GEMM family (v_mfma_f32_32x32x2f32) against the CPU oracle.

Bar (north star): relative Frobenius error <= 1e-4 against the double-precision
restatement of ai/core/matrix.lua's loops, on identical fp32-representable
inputs.  Large shapes are checked against numpy float64 '@' (an independent
library product; the oracle's loops agree with it to 1e-12, tests/test_oracle.py).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from lanternl_amd import device, kernels
from tests.gpu_util import announce, f32, rel_fro, to_dev

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module", autouse=True)
def _dev():
    device.init(0)
    yield


def _gemm(ta, tb, a, b, alpha=1.0, beta=0.0, c0=None):
    A, B = to_dev(a), to_dev(b)
    m = a.shape[1] if ta else a.shape[0]
    n = b.shape[0] if tb else b.shape[1]
    C = to_dev(c0) if c0 is not None else device.Buffer((m, n))
    kernels.sgemm(A, B, C, transa=ta, transb=tb, alpha=alpha, beta=beta)
    device.sync()
    return C.download().astype(np.float64)


@pytest.mark.parametrize("m,k,n", [(256, 128, 256),          # config C1
                                   (37, 53, 41), (128, 96, 160),  # tests/test.lua:42,65
                                   (1, 1, 1), (3, 5, 7), (64, 64, 16), (65, 33, 129),
                                   (1, 300, 257), (200, 1, 130)])
def test_gemm_family_vs_oracle(m, k, n):
    announce("gemm family", m, k, n)
    rng = np.random.default_rng(1000 + m * 7 + k * 3 + n)
    a = f32(rng.uniform(-1, 1, (m, k)))
    b = f32(rng.uniform(-1, 1, (k, n)))
    ref = O.mm(a, b)                                       # matrix.lua:514-539
    assert rel_fro(_gemm(False, False, a, b), ref) <= TOL
    bt = np.ascontiguousarray(b.T)                         # B stored n x k
    assert rel_fro(_gemm(False, True, a, bt), O.matmul_nt(a, bt)) <= TOL
    at = np.ascontiguousarray(a.T)                         # A stored k x m: C = at^T . b
    assert rel_fro(_gemm(True, False, at, b), O.matmul_tn(at, b)) <= TOL
    assert rel_fro(_gemm(True, True, at, bt), ref) <= TOL


@pytest.mark.parametrize("m,k,n", [(64, 4096, 4096), (40, 2500, 1100), (1000, 8192, 600)])
def test_gemm_split_band_on_four_wave_sets(m, k, n):
    """Few 64x64 tiles with long K, split over K into slices of 1024 or more
    on four wave sets (33..64 rows: one tile band; 1000 x 600 x 8192: 160
    tiles in 2 slices), slices summed in order by the reduce, all four
    transposition variants, ragged M, N and K."""
    announce("gemm split band", m, k, n)
    rng = np.random.default_rng(m * 3 + k + n)
    a = f32(rng.uniform(-1, 1, (m, k)))
    b = f32(rng.uniform(-1, 1, (k, n)))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    at, bt = np.ascontiguousarray(a.T), np.ascontiguousarray(b.T)
    for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
        got = _gemm(bool(ta), bool(tb), at if ta else a, bt if tb else b)
        assert rel_fro(got, ref) <= TOL, (ta, tb)


@pytest.mark.parametrize("m,k,n", [(1024, 1024, 1024), (1000, 777, 1030), (2048, 1024, 1024), (512, 128, 2000),
                                   (500, 100, 2040), (500, 1024, 2000), (510, 512, 2044), (60, 2048, 2000)])
def test_gemm_two_wave_set_tiles(m, k, n):
    """Mid-size products with long K on one or two 64x64 tiles per CU (two
    wave sets taking every second K chunk; K = 777 ragged with an odd chunk
    count), short K at one tile per CU on two wave sets as well (the C2 tied
    head 512x2000x128; K = 100 ragged),
    all four transposition variants, and alpha / beta.  Whole 32-deep chunks
    take the unconditional-load form with rows and columns past M and N
    clamped: 500x1024x2000 (edge tiles in M and N), 510x512x2044 (M % 4 != 0:
    the K-major-A variants keep the guarded loads), 60x2048x2000 (the split
    64-row band)."""
    announce("gemm two wave sets", m, k, n)
    rng = np.random.default_rng(m + k + n)
    a = f32(rng.uniform(-1, 1, (m, k)))
    b = f32(rng.uniform(-1, 1, (k, n)))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    at, bt = np.ascontiguousarray(a.T), np.ascontiguousarray(b.T)
    for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
        got = _gemm(bool(ta), bool(tb), at if ta else a, bt if tb else b)
        assert rel_fro(got, ref) <= TOL, (ta, tb)
    c0 = f32(rng.uniform(-1, 1, (m, n)))
    got = _gemm(False, False, a, b, alpha=0.5, beta=-2.0, c0=c0)
    assert rel_fro(got, 0.5 * ref - 2.0 * c0.astype(np.float64)) <= TOL


@pytest.mark.parametrize("m,k,n", [(1536, 1536, 1536), (1500, 777, 1700), (1536, 256, 1536), (1600, 800, 1600)])
def test_gemm_one_wave_set_tiles(m, k, n):
    """Products with more 64x64 tiles than two per CU below the big-tile sizes
    (or short K) on the wave-set kernel with one set: whole-chunk loads two
    chunks ahead, or the guarded loads for K = 777; all four transposition
    variants and alpha / beta, against float64."""
    announce("gemm one wave set", m, k, n)
    rng = np.random.default_rng(m + 3 * k + n)
    a = f32(rng.uniform(-1, 1, (m, k)))
    b = f32(rng.uniform(-1, 1, (k, n)))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    at, bt = np.ascontiguousarray(a.T), np.ascontiguousarray(b.T)
    for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
        got = _gemm(bool(ta), bool(tb), at if ta else a, bt if tb else b)
        assert rel_fro(got, ref) <= TOL, (ta, tb)
    c0 = f32(rng.uniform(-1, 1, (m, n)))
    got = _gemm(False, False, a, b, alpha=0.5, beta=-2.0, c0=c0)
    assert rel_fro(got, 0.5 * ref - 2.0 * c0.astype(np.float64)) <= TOL


@pytest.mark.parametrize("m,k,n", [(512, 32000, 128), (500, 20000, 130), (300, 20000, 200)])
def test_gemm_big_tiles_split_over_k(m, k, n):
    """Few 128x128 tiles over a long K (C3 dhidden 512x128x32000): the big-tile
    kernel split over K into one slice per CU's worth of tiles, the slices
    summed in order by the reduce; all four transposition variants, ragged M,
    N and K, and alpha / beta."""
    announce("gemm big tiles split", m, k, n)
    rng = np.random.default_rng(m + 7 * k + n)
    a = f32(rng.uniform(-1, 1, (m, k)))
    b = f32(rng.uniform(-1, 1, (k, n)))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    at, bt = np.ascontiguousarray(a.T), np.ascontiguousarray(b.T)
    for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
        got = _gemm(bool(ta), bool(tb), at if ta else a, bt if tb else b)
        assert rel_fro(got, ref) <= TOL, (ta, tb)
    c0 = f32(rng.uniform(-1, 1, (m, n)))
    got = _gemm(False, True, a, bt, alpha=0.5, beta=-2.0, c0=c0)
    assert rel_fro(got, 0.5 * ref - 2.0 * c0.astype(np.float64)) <= TOL


def test_gemm_c1_all_variants_bitwise_stable():
    """Config C1: A 256x128, B 128x256; the three products agree with the oracle
    and with each other (A.B = (A^T)^T.B = A.(B^T)^T) to fp32 rounding."""
    announce("gemm C1")
    rng = np.random.default_rng(1)
    a = f32(rng.uniform(-1, 1, (256, 128)))
    b = f32(rng.uniform(-1, 1, (128, 256)))
    nn = _gemm(False, False, a, b)
    tn = _gemm(True, False, np.ascontiguousarray(a.T), b)
    nt = _gemm(False, True, a, np.ascontiguousarray(b.T))
    ref = O.mm(a, b)
    for c in (nn, tn, nt):
        assert rel_fro(c, ref) <= TOL
    # same accumulation order on every variant -> identical fp32 results
    assert np.array_equal(nn, tn) and np.array_equal(nn, nt)


def test_gemm_alpha_beta_and_nan_in_c():
    announce("gemm alpha/beta")
    rng = np.random.default_rng(2)
    a = f32(rng.uniform(-1, 1, (70, 90)))
    b = f32(rng.uniform(-1, 1, (90, 50)))
    ref = O.mm(a, b)
    # tests/test.lua:115-122: beta = 1 on top of the same product doubles it
    c1 = _gemm(False, False, a, b)
    c2 = _gemm(False, False, a, b, beta=1.0, c0=c1)
    assert rel_fro(c2, 2 * ref) <= TOL
    c0 = f32(rng.uniform(-1, 1, (70, 50)))
    c3 = _gemm(False, False, a, b, alpha=-0.5, beta=0.25, c0=c0)
    assert rel_fro(c3, -0.5 * ref + 0.25 * c0) <= TOL
    # beta == 0 never reads C
    cnan = np.full((70, 50), np.nan)
    c4 = _gemm(False, False, a, b, beta=0.0, c0=cnan)
    assert np.isfinite(c4).all() and rel_fro(c4, ref) <= TOL


def test_gemm_k_zero_scales_c():
    announce("gemm k=0")
    c0 = np.arange(12, dtype=np.float64).reshape(3, 4)
    C = to_dev(c0)
    A = device.Buffer((3, 1)); B = device.Buffer((1, 4))
    kernels.sgemm_raw(0, 0, 3, 4, 0, 1.0, A.ptr, 1, B.ptr, 4, 2.0, C.ptr, 4)
    device.sync()
    assert np.array_equal(C.download(), 2 * c0)


def test_gemm_unaligned_leading_dims_and_views():
    """Strided sub-matrix views (ld > cols, odd offsets) take the scalar path."""
    announce("gemm strided views")
    rng = np.random.default_rng(3)
    big_a = f32(rng.uniform(-1, 1, (50, 77)))
    big_b = f32(rng.uniform(-1, 1, (61, 45)))
    A, B = to_dev(big_a), to_dev(big_b)
    m, k, n = 33, 41, 29
    a = big_a[2:2 + m, 3:3 + k]
    b = big_b[5:5 + k, 1:1 + n]
    C = device.Buffer((m, n))
    kernels.sgemm_raw(0, 0, m, n, k, 1.0, A.offset(2 * 77 + 3), 77, B.offset(5 * 45 + 1), 45, 0.0, C.ptr, n)
    device.sync()
    assert rel_fro(C.download(), O.mm(np.ascontiguousarray(a), np.ascontiguousarray(b))) <= TOL


def test_gemm_strided_batched_per_head_qk():
    """Per-head Q.K^T through strides (tests/test.lua:128-160: T=8, H=3, hd=4),
    plus a larger causal-attention shape (T=64, H=8, hd=16)."""
    for T, H, hd in ((8, 3, 4), (64, 8, 16)):
        announce("gemm batched qk", T, H, hd)
        rng = np.random.default_rng(T + H)
        q = f32(rng.uniform(-1, 1, (T, H * hd)))
        k = f32(rng.uniform(-1, 1, (T, H * hd)))
        Q, K = to_dev(q), to_dev(k)
        S = device.Buffer((H, T, T))
        kernels.sgemm_strided_batched(0, 1, T, T, hd, 1.0, Q.ptr, H * hd, hd, K.ptr, H * hd, hd,
                                      0.0, S.ptr, T, T * T, H)
        device.sync()
        s = S.download().astype(np.float64)
        for h in range(H):
            qh = np.ascontiguousarray(q[:, h * hd:(h + 1) * hd])
            kh = np.ascontiguousarray(k[:, h * hd:(h + 1) * hd])
            assert rel_fro(s[h], O.matmul_nt(qh, kh)) <= TOL


@pytest.mark.parametrize("n", [1024, 2048, 4096])
def test_gemm_square_large(n):
    """Config C5 square shapes (1024^3, 2048^3, 4096^3), all three products, vs
    numpy float64.  2048^3 runs 64 256x256 tiles split four ways over K."""
    announce("gemm square", n)
    rng = np.random.default_rng(n)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    A, B, C = to_dev(a), to_dev(b), device.Buffer((n, n))
    for ta, tb, aa, bb in ((0, 0, A, B), (1, 0, None, B), (0, 1, A, None)):
        if ta:
            aa = to_dev(np.ascontiguousarray(a.T))
        if tb:
            bb = to_dev(np.ascontiguousarray(b.T))
        kernels.sgemm(aa, bb, C, transa=ta, transb=tb)
        device.sync()
        assert rel_fro(C.download(), ref) <= TOL, (ta, tb)


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_gemm_square_8192(ta, tb):
    """Config C5's largest square shape, 8192^3, for A.B, A^T.B and A.B^T.

    A full float64 product would take minutes on the host, so two checks
    cover it:
      * 256 whole rows of C, drawn at random over every row band, against
        float64 (relative Frobenius <= 1e-4);
      * a Freivalds check of every row of C: with two random vectors x,
        C.x against op(A).(op(B).x) in float64, row by row, relative to
        |C_i| |x|.  A single wrong element of size e in row i moves that row's
        residual by about e |x_j|; fp32 rounding moves it by ~1e-8 of the
        scale (2.3e-8 measured for numpy's fp32 product at 4096^3), so the
        1e-6 bar catches any element wrong by more than ~0.5 (entries of C
        are ~ sqrt(8192/9) = 30 in size).
    """
    n = 8192
    announce("gemm square 8192", ta, tb)
    rng = np.random.default_rng(8192 + 2 * ta + tb)
    a = rng.uniform(-1, 1, (n, n)).astype(np.float32)     # stored operand (k x m when ta)
    b = rng.uniform(-1, 1, (n, n)).astype(np.float32)     # stored operand (n x k when tb)
    A, B, C = to_dev(a), to_dev(b), device.Buffer((n, n))
    kernels.sgemm(A, B, C, transa=ta, transb=tb)
    device.sync()
    del A, B
    c = C.download()
    del C
    opa = a.T if ta else a            # op(A), views
    opb = b.T if tb else b
    rows = np.sort(rng.choice(n, 256, replace=False))
    ref_rows = opa[rows].astype(np.float64) @ opb.astype(np.float64)
    assert rel_fro(c[rows], ref_rows) <= TOL
    x = rng.standard_normal((n, 2))
    bx = opb.astype(np.float64) @ x
    abx = opa.astype(np.float64) @ bx
    cx = c.astype(np.float64) @ x
    scale = np.linalg.norm(c.astype(np.float64), axis=1)[:, None] * np.linalg.norm(x, axis=0)[None, :]
    worst = float(np.max(np.abs(cx - abx) / scale))
    assert worst <= 1e-6, worst


@pytest.mark.parametrize("m", [1, 16, 64])
def test_gemm_skinny(m):
    """Config C5 skinny shapes: M in {1,16,64}, K=N=4096."""
    announce("gemm skinny", m)
    rng = np.random.default_rng(77 + m)
    a = rng.uniform(-1, 1, (m, 4096)).astype(np.float32)
    b = rng.uniform(-1, 1, (4096, 4096)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    C = device.Buffer((m, 4096))
    kernels.sgemm(to_dev(a), to_dev(b), C)
    device.sync()
    assert rel_fro(C.download(), ref) <= TOL


def test_sgemm_rejects_bad_arguments_without_launch():
    from lanternl_amd._lib import LanternlHipError
    A = device.Buffer((4, 4))
    with pytest.raises(LanternlHipError, match="lda"):
        kernels.sgemm_raw(0, 0, 4, 4, 4, 1.0, A.ptr, 2, A.ptr, 4, 0.0, A.ptr, 4)
    with pytest.raises(LanternlHipError, match="negative"):
        kernels.sgemm_raw(0, 0, -1, 4, 4, 1.0, A.ptr, 4, A.ptr, 4, 0.0, A.ptr, 4)
    with pytest.raises(LanternlHipError, match="NULL"):
        kernels.sgemm_raw(0, 0, 4, 4, 4, 1.0, None, 4, A.ptr, 4, 0.0, A.ptr, 4)


# ------------------------------------------------------- flat-table backend contract
def test_adapter_legacy_flat_matmul_known_answer():
    """tests/test.lua:445-449 and tests/core_test.lua:31-34 through the backend module."""
    announce("adapter known answers")
    from lanternl_amd import backend
    assert backend.available, backend.reason
    assert backend.matmul([1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 1, 1, 1], 2) == [4, 5, 10, 11]
    assert backend.matmul([1, 2, 3, 4], 2, 2, [5, 6, 7, 8], 2) == [19, 22, 43, 50]
    # nt: a(2x3) . b(2x3)^T ; tn: a(2x3)^T . b(2x2)
    assert backend.matmul_nt([1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 0, 1, 1], 2) == [1, 5, 4, 11]
    assert backend.matmul_tn([1, 2, 3, 4, 5, 6], 2, 3, [1, 0, 0, 1], 2) == [1, 4, 2, 5, 3, 6]


def test_matrix_registry_offloads_all_three_products():
    """ai.Matrix with the backend forced: multiply / matmul_nt / matmul_tn all run on
    the GPU (last_backend) and match the Lua loops (oracle) at config C1."""
    announce("matrix registry C1")
    from lanternl_amd import matrix as MX
    MX.reset_backends()
    assert MX.use("luatl_adapter") == "luatl_adapter"
    try:
        rng = np.random.default_rng(5)
        a = f32(rng.uniform(-1, 1, (256, 128)))
        b = f32(rng.uniform(-1, 1, (128, 256)))
        r = MX.multiply(MX.Matrix.from_numpy(a), MX.Matrix.from_numpy(b))
        assert MX.last_backend == "luatl_adapter"
        assert rel_fro(r.to_numpy(), O.mm(a, b)) <= TOL
        bt = np.ascontiguousarray(b.T)
        r = MX.matmul_nt(MX.Matrix.from_numpy(a), MX.Matrix.from_numpy(bt))
        assert MX.last_backend == "luatl_adapter"
        assert rel_fro(r.to_numpy(), O.matmul_nt(a, bt)) <= TOL
        x = f32(rng.uniform(-1, 1, (128, 256)))   # m x k
        y = f32(rng.uniform(-1, 1, (128, 256)))   # m x n
        r = MX.matmul_tn(MX.Matrix.from_numpy(x), MX.Matrix.from_numpy(y))
        assert MX.last_backend == "luatl_adapter"
        assert rel_fro(r.to_numpy(), O.matmul_tn(x, y)) <= TOL
    finally:
        MX.use("auto")


def test_matmul_host_accumulate_in_double():
    announce("matmul_host acc")
    from lanternl_amd._lib import call
    rng = np.random.default_rng(9)
    a = f32(rng.uniform(-1, 1, (20, 30)))
    b = f32(rng.uniform(-1, 1, (30, 10)))
    c = rng.uniform(-1, 1, (20, 10))            # arbitrary doubles
    expect = c + O.mm(a, b)
    out = c.copy()
    call("lhip_matmul_host", 0, a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p),
         out.ctypes.data_as(ctypes.c_void_p), 20, 30, 10, 1)
    assert rel_fro(out, expect) <= TOL


def test_matmul_host_with_workers_not_spinning():
    """lhip_set_host_spin(0): the conversion workers sleep at once after each
    call; results are unchanged (C1, all three products), the old value comes
    back, and out-of-range values are refused."""
    announce("matmul_host spin 0")
    from lanternl_amd._lib import LanternlHipError, call
    prev = ctypes.c_int()
    call("lhip_set_host_spin", 0, ctypes.byref(prev))
    try:
        rng = np.random.default_rng(21)
        a = f32(rng.uniform(-1, 1, (256, 128)))
        b = f32(rng.uniform(-1, 1, (128, 256)))
        for op, bb, ref in ((0, b, O.mm(a, b)), (1, np.ascontiguousarray(b.T), O.mm(a, b)),
                            (2, f32(rng.uniform(-1, 1, (256, 256))), None)):
            if op == 2:
                ref = O.matmul_tn(a, bb)
            rows, n = (128, 256) if op == 2 else (256, 256)
            out = np.empty((rows, n))
            for _ in range(3):    # back to back: the workers sleep and wake each time
                call("lhip_matmul_host", op, a.ctypes.data_as(ctypes.c_void_p), bb.ctypes.data_as(ctypes.c_void_p),
                     out.ctypes.data_as(ctypes.c_void_p), 256, 128, 256, 0)
                assert rel_fro(out, ref) <= TOL
        with pytest.raises(LanternlHipError, match="outside"):
            call("lhip_set_host_spin", -1, None)
        got = ctypes.c_int()
        call("lhip_set_host_spin", 0, ctypes.byref(got))
        assert got.value == 0
    finally:
        call("lhip_set_host_spin", prev.value, None)
    assert prev.value == 1000


def test_matmul_host_small_calls_back_to_back():
    """Small calls (under 1 Mi elements) convert on the calling thread and the
    pool's spinning workers: 240 calls of random shapes (one to four parts per
    conversion), ops and accumulate flags, with pauses past the workers' spin
    window every 40 calls, each against the float64 product of the
    fp32-rounded inputs."""
    announce("matmul_host small calls")
    import time
    from lanternl_amd._lib import call
    rng = np.random.default_rng(77)
    for i in range(240):
        op, acc = int(rng.integers(0, 3)), int(rng.integers(0, 2))
        m, k, n = (int(x) for x in rng.integers(1, 300, 3))
        a = rng.uniform(-1, 1, (m, k))
        b = rng.uniform(-1, 1, {0: (k, n), 1: (n, k), 2: (m, n)}[op])
        a32, b32 = a.astype(np.float32).astype(np.float64), b.astype(np.float32).astype(np.float64)
        ref = {0: lambda: a32 @ b32, 1: lambda: a32 @ b32.T, 2: lambda: a32.T @ b32}[op]()
        c0 = rng.uniform(-1, 1, ref.shape)
        out = c0.copy()
        call("lhip_matmul_host", op, a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p),
             out.ctypes.data_as(ctypes.c_void_p), m, k, n, acc)
        assert rel_fro(out, ref + c0 if acc else ref) <= TOL, (i, op, m, k, n, acc)
        if i % 40 == 39:
            time.sleep(0.003)


@pytest.mark.parametrize("op,m,k,n,acc", [(0, 2048, 2304, 2048, 0), (1, 1500, 1024, 1300, 1), (2, 2100, 1000, 900, 0)])
def test_matmul_host_threaded_chunks(op, m, k, n, acc):
    """Calls large enough for the threaded, chunked host path (conversions on
    the host pool, 16 MiB chunks: op 0 has two upload chunks per operand and
    two download chunks) against float64 products of the fp32-rounded inputs."""
    announce("matmul_host threaded", op, m, k, n, acc)
    from lanternl_amd._lib import call
    rng = np.random.default_rng(40 + op)
    a = rng.uniform(-1, 1, (m, k))
    b = rng.uniform(-1, 1, {0: (k, n), 1: (n, k), 2: (m, n)}[op])
    a32, b32 = a.astype(np.float32).astype(np.float64), b.astype(np.float32).astype(np.float64)
    ref = {0: lambda: a32 @ b32, 1: lambda: a32 @ b32.T, 2: lambda: a32.T @ b32}[op]()
    c0 = rng.uniform(-1, 1, ref.shape)
    out = c0.copy()
    call("lhip_matmul_host", op, a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p),
         out.ctypes.data_as(ctypes.c_void_p), m, k, n, acc)
    assert rel_fro(out, ref + c0 if acc else ref) <= TOL
    # a second call reuses the staging and the pool
    out2 = np.zeros_like(ref)
    call("lhip_matmul_host", op, a.ctypes.data_as(ctypes.c_void_p), b.ctypes.data_as(ctypes.c_void_p),
         out2.ctypes.data_as(ctypes.c_void_p), m, k, n, 0)
    assert rel_fro(out2, ref) <= TOL


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_gemm_c3_lm_head_shapes(ta, tb):
    """Config C3: logits = hidden(512x128) . W(128x32000); dW = hidden^T . dlogits;
    dhidden = dlogits . W^T (K = 32000, the split-K path)."""
    announce("gemm C3", ta, tb)
    rng = np.random.default_rng(30 + 2 * ta + tb)
    hidden = rng.standard_normal((512, 128)).astype(np.float32)
    W = (rng.standard_normal((128, 32000)) * 0.02).astype(np.float32)
    dlog = (rng.standard_normal((512, 32000)) * 1e-3).astype(np.float32)
    if (ta, tb) == (0, 0):
        a, b, ref = hidden, W, hidden.astype(np.float64) @ W.astype(np.float64)
    elif (ta, tb) == (1, 0):
        a, b, ref = hidden, dlog, hidden.T.astype(np.float64) @ dlog.astype(np.float64)
    else:
        a, b, ref = dlog, W, dlog.astype(np.float64) @ W.T.astype(np.float64)
    got = _gemm(bool(ta), bool(tb), a, b)
    assert rel_fro(got, ref) <= TOL


@pytest.mark.parametrize("m,n,k,batch", [(512, 128, 2000, 1), (128, 128, 4096, 3), (64, 64, 1000, 2),
                                         (96, 64, 1100, 2), (512, 512, 2048, 1), (33, 70, 999, 1),
                                         (1, 4096, 4096, 1), (2048, 2048, 1024, 1)])
def test_gemm_split_k_alpha_beta_batched(m, n, k, batch):
    """Long-K shapes with few output tiles: the 256x256 (2048 x 2048), 64x64 and
    32x32 kernels split K (alpha/beta apply once, after the ordered sum of the
    slices); the 16x16 kernel walks long K in software-pipelined passes."""
    announce("gemm split-k", m, n, k, batch)
    rng = np.random.default_rng(m + n + k)
    a = f32(rng.uniform(-1, 1, (batch, m, k)))
    b = f32(rng.uniform(-1, 1, (batch, k, n)))
    c0 = f32(rng.uniform(-1, 1, (batch, m, n)))
    A, B, C = to_dev(a), to_dev(b), to_dev(c0)
    kernels.sgemm_strided_batched(0, 0, m, n, k, 0.5, A.ptr, k, m * k, B.ptr, n, k * n, -2.0, C.ptr, n, m * n, batch)
    device.sync()
    got = C.download().astype(np.float64)
    for z in range(batch):
        assert rel_fro(got[z], 0.5 * (a[z] @ b[z]) - 2.0 * c0[z]) <= TOL
    # deterministic: the same call twice gives bit-identical results
    C2 = to_dev(c0)
    kernels.sgemm_strided_batched(0, 0, m, n, k, 0.5, A.ptr, k, m * k, B.ptr, n, k * n, -2.0, C2.ptr, n, m * n, batch)
    device.sync()
    assert np.array_equal(C2.download(), C.download())


def _ref_op(x, t):
    return x.T if t else x


@pytest.mark.parametrize("ta,tb,m,n,k,count", [
    (0, 1, 512, 128, 256, 2),     # C2 dh2 = dz1.W1^T + du.W3^T
    (0, 1, 512, 128, 128, 3),     # C2 dh = dq.Wq^T + dk.Wk^T + dv.Wv^T
    (0, 0, 37, 53, 40, 3),        # ragged tiles, NN
    (0, 1, 45, 19, 10, 2),        # K not a multiple of 4: block by block
    (1, 0, 64, 48, 32, 2),        # transposed A: block by block
    (0, 0, 1024, 1024, 256, 2),   # large: the 128x128 kernel, block by block
    (0, 1, 300, 200, 64, 1),      # count 1 = a plain GEMM
])
def test_gemm_batched_reduce_vs_oracle(ta, tb, m, n, k, count):
    """lhip_sgemm_batched_reduce: C = alpha * sum_j op(A_j) op(B_j) + beta * C, checked
    against the oracle's products summed in double (matrix.lua mm / matmul_nt /
    matmul_tn with acc, the CPU backward's accumulation)."""
    announce("gemm batch-reduce", ta, tb, m, n, k, count)
    rng = np.random.default_rng(m * 7 + n + k + count)
    a_shape = (k, m) if ta else (m, k)
    b_shape = (n, k) if tb else (k, n)
    a = f32(rng.uniform(-1, 1, (count,) + a_shape))
    b = f32(rng.uniform(-1, 1, (count,) + b_shape))
    c0 = f32(rng.uniform(-1, 1, (m, n)))
    alpha, beta = 0.75, 0.5
    A, B, C = to_dev(a), to_dev(b), to_dev(c0)
    sa, sb = int(np.prod(a_shape)), int(np.prod(b_shape))
    kernels.sgemm_batched_reduce(ta, tb, m, n, k, alpha, A.ptr, a_shape[1], sa, B.ptr, b_shape[1], sb, beta,
                                 C.ptr, n, count)
    device.sync()
    got = C.download().astype(np.float64)
    ref = beta * c0.astype(np.float64)
    acc = np.zeros((m, n))
    for j in range(count):
        aj, bj = a[j].astype(np.float64), b[j].astype(np.float64)
        if ta:
            acc += O.matmul_tn(aj, bj) if not tb else _ref_op(aj, 1) @ _ref_op(bj, 1)
        elif tb:
            acc += O.matmul_nt(aj, bj)
        else:
            acc += O.mm(aj, bj)
    ref += alpha * acc
    assert rel_fro(got, ref) <= TOL


def test_gemm_batched_reduce_rejects_bad_count():
    from lanternl_amd._lib import LanternlHipError
    A = device.Buffer((4, 4))
    with pytest.raises(LanternlHipError):
        kernels.sgemm_batched_reduce(0, 0, 4, 4, 4, 1.0, A.ptr, 4, 16, A.ptr, 4, 16, 0.0, A.ptr, 4, 0)


@pytest.mark.parametrize("m,n,k,batch,ld_pad", [(4096, 4096, 96, 1, 0),     # every tile full
                                                (4000, 4100, 203, 1, 0),   # ragged M, N and K
                                                (4096, 4096, 64, 1, 1),    # ld % 4 != 0: scalar loads
                                                (1024, 1024, 80, 16, 0),   # 16 x 16 tiles per batch
                                                # 128x128 tiles on the same kernel
                                                (2048, 2048, 96, 1, 0),    # every tile full
                                                (2000, 2100, 203, 1, 0),   # ragged M, N and K
                                                (2048, 2048, 64, 1, 1),    # scalar loads
                                                (512, 512, 80, 16, 0),     # 4 x 4 tiles per batch
                                                (128, 32000, 96, 1, 0)])   # one row of tiles (C3 dW shape)
def test_gemm_256_tile_path(m, n, k, batch, ld_pad):
    """Problems with at least one 256x256 output tile per CU, and those with
    fewer but about one 128x128 tile per CU or more (the same kernel on
    128x128 tiles): all four operand layouts, alpha/beta, vs numpy float64 on
    each batch entry."""
    announce("gemm 256 tiles", m, n, k, batch, ld_pad)
    rng = np.random.default_rng(m + n + k + batch + ld_pad)
    a = rng.uniform(-1, 1, (batch, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (batch, k, n)).astype(np.float32)
    c0 = rng.uniform(-1, 1, (batch, m, n)).astype(np.float32)
    ref = 0.5 * np.matmul(a.astype(np.float64), b.astype(np.float64)) - 2.0 * c0
    for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
        sa = np.ascontiguousarray(a.transpose(0, 2, 1)) if ta else a
        sb = np.ascontiguousarray(b.transpose(0, 2, 1)) if tb else b
        lda, ldb, ldc = sa.shape[2] + ld_pad, sb.shape[2] + ld_pad, n + ld_pad
        pa = np.zeros((batch, sa.shape[1], lda), np.float32)
        pa[:, :, :sa.shape[2]] = sa
        pb = np.zeros((batch, sb.shape[1], ldb), np.float32)
        pb[:, :, :sb.shape[2]] = sb
        pc = np.full((batch, m, ldc), np.nan, np.float32)
        pc[:, :, :n] = c0
        A, B, C = to_dev(pa), to_dev(pb), to_dev(pc)
        kernels.sgemm_strided_batched(ta, tb, m, n, k, 0.5, A.ptr, lda, pa[0].size, B.ptr, ldb, pb[0].size,
                                      -2.0, C.ptr, ldc, pc[0].size, batch)
        device.sync()
        got = C.download().reshape(batch, m, ldc)
        for z in range(batch):
            assert rel_fro(got[z, :, :n], ref[z]) <= TOL, (ta, tb, z)
        if ld_pad:
            assert np.isnan(got[:, :, n:]).all(), "wrote outside the n columns"


# ------------------------------------------------------------ skinny products
# M <= 64 with B stored K x N take the streaming kernel (one pass over B,
# K split into slices summed in order; 3..64 rows on the matrix cores in one to
# four 16-row groups); edge columns, unaligned leading dimensions, transposed
# A, alpha/beta and K shorter than a slice are covered.
@pytest.mark.parametrize("m,k,n", [(1, 4096, 4096), (16, 4096, 4096), (1, 7, 256), (2, 64, 300),
                                   (3, 1000, 513), (5, 333, 1024), (8, 4097, 257), (13, 129, 777),
                                   (16, 64, 256), (11, 2, 4096), (17, 300, 257), (33, 512, 300),
                                   (48, 1000, 1024), (64, 4096, 4096), (61, 77, 4097), (64, 3, 256)])
def test_gemm_skinny_vs_oracle(m, k, n):
    announce("gemm skinny", m, k, n)
    rng = np.random.default_rng(7000 + m * 11 + k + n)
    a = f32(rng.uniform(-1, 1, (m, k)))
    b = f32(rng.uniform(-1, 1, (k, n)))
    ref = a @ b if k * n > 1 << 22 else O.mm(a, b)
    assert rel_fro(_gemm(False, False, a, b), ref) <= TOL
    at = np.ascontiguousarray(a.T)
    assert rel_fro(_gemm(True, False, at, b), ref) <= TOL
    c0 = f32(rng.uniform(-1, 1, (m, n)))
    assert rel_fro(_gemm(False, False, a, b, alpha=0.5, beta=-2.0, c0=c0), 0.5 * ref - 2.0 * c0) <= TOL


def test_gemm_skinny_strided_views_and_matrix_multiply_gate():
    """Skinny shapes through strided views (scalar B loads) and ldc > n."""
    announce("gemm skinny strided")
    rng = np.random.default_rng(71)
    big_a = f32(rng.uniform(-1, 1, (9, 803)))
    big_b = f32(rng.uniform(-1, 1, (801, 611)))
    A, B = to_dev(big_a), to_dev(big_b)
    m, k, n = 7, 799, 601
    C = device.Buffer((m, 605))
    kernels.sgemm_raw(0, 0, m, n, k, 1.0, A.offset(1 * 803 + 2), 803, B.offset(1 * 611 + 3), 611, 0.0, C.ptr, 605)
    device.sync()
    got = C.download()[:, :n]
    ref = O.mm(np.ascontiguousarray(big_a[1:1 + m, 2:2 + k]), np.ascontiguousarray(big_b[1:1 + k, 3:3 + n]))
    assert rel_fro(got, ref) <= TOL


def _sweep_cases(rng, count):
    """Shapes that take every branch of the dispatcher, then random ones
    (log-uniform sizes, at most 1.5 Gflop each)."""
    cases = [(1, 4096, 3000), (2, 300, 4000), (16, 3000, 2000), (48, 2048, 4096), (64, 1024, 2048),
             (1024, 1024, 1024), (1000, 1030, 600), (512, 2000, 128), (2048, 1536, 512), (300, 2500, 64),
             (1536, 1536, 256), (257, 129, 1), (3, 5, 7)]
    while len(cases) < count:
        m, n, k = (int(np.exp(rng.uniform(0, np.log(x)))) for x in (2600, 2600, 4100))
        if m * n * k <= 750_000_000:
            cases.append((m, n, k))
    return cases


def test_gemm_random_dispatch_sweep():
    """Seeded random products over every dispatch branch (skinny, split band,
    16x16 / 32x32 / 64x64 tiles on one, two and four wave sets, 128x128 and
    256x256 tiles, split-K with its reduce), each with random transposes,
    alpha and beta, leading dimensions padded past the logical rows and
    operands that start one element past a 16-byte boundary; against float64
    at the GEMM bar, and every padding element of C left as it was."""
    rng = np.random.default_rng(20261202)
    for i, (m, n, k) in enumerate(_sweep_cases(rng, 44)):
        ta, tb = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        pad = [int(rng.choice([0, 0, 3, 4, 9])) for _ in range(3)]
        off = [int(rng.integers(0, 2)) for _ in range(3)]
        alpha = float(rng.choice([1.0, 0.5, -1.25]))
        beta = float(rng.choice([0.0, 0.0, 1.0, -0.5]))
        announce("gemm sweep", i, (m, n, k), "ta" if ta else "", "tb" if tb else "", pad, off, alpha, beta)
        a = f32(rng.uniform(-1, 1, (m, k)))
        b = f32(rng.uniform(-1, 1, (k, n)))
        c0 = f32(rng.uniform(-1, 1, (m, n)))
        sa = np.ascontiguousarray(a.T) if ta else a          # stored operand
        sb = np.ascontiguousarray(b.T) if tb else b
        lda, ldb, ldc = sa.shape[1] + pad[0], sb.shape[1] + pad[1], n + pad[2]
        bufs = []
        for x, ld, o in ((sa, lda, off[0]), (sb, ldb, off[1]), (c0, ldc, off[2])):
            store = np.full(o + x.shape[0] * ld + 4, 7.0, np.float32)
            store[o:o + x.shape[0] * ld].reshape(x.shape[0], ld)[:, :x.shape[1]] = x
            bufs.append((device.Buffer.from_numpy(store), store, o, ld))
        (A, _, oa, _), (B, _, ob, _), (C, cst, oc, _) = bufs
        kernels.sgemm_raw(int(ta), int(tb), m, n, k, alpha, A.offset(oa), lda, B.offset(ob), ldb, beta,
                          C.offset(oc), ldc)
        device.sync()
        out = C.download()
        got = out[oc:oc + m * ldc].reshape(m, ldc)
        ref = alpha * (a.astype(np.float64) @ b.astype(np.float64)) + beta * c0.astype(np.float64)
        assert rel_fro(got[:, :n], ref) <= TOL, (i, m, n, k, ta, tb)
        untouched = np.ones(out.shape, bool)
        untouched[oc:oc + m * ldc].reshape(m, ldc)[:, :n] = False
        assert np.array_equal(out[untouched], cst[untouched]), ("C written outside its rows", i, m, n, k)
