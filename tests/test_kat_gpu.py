"""The reference's forward known answers (tests/check_ops.c:69-182) and the
error bounds of the device's transcendental paths, run through the
product's own kernels.

``tests/kat/libcngpt_kat.so`` is a test-only C entry layer over the
launchers of ``libcngpt_hip.so`` (the same compiled kernels the forward
calls); it adds nothing to ``include/``.

Known answers (check_ops.c), each through every product variant that can
compute it:
- linear 2x2 -> [[3, 3], [4, 4]] (:69-82): the decode product (M <= 8), the
  weight-streaming product (M <= 64) and the 128 x 128 MFMA tiles with K = 4
  (register-staged), 16 and 32 (direct-to-LDS), K zero-padded (zeros do not
  change the answer) and the two rows embedded in a 130-row product;
- LayerNorm of [1, 2, 3, 4] (:118-136);
- GELU at 0, 1, -1, 2 (:146-157), through the bias+GELU epilogue of the
  identity product (x * 1 + 0 is exact);
- softmax of [1, 2, 3] and [100, 100, 100] (:165-182), through the fused
  causal attention kernel and the one-query-row (decode) kernel with values
  that are one-hot rows, so the output row is the probability row.

Error bounds (u = 2^-24, gamma_n = n u):
- GELU: the device evaluates x / (1 + exp(-2v)), v = sqrt(2/pi)(x +
  0.044715 x^3). v carries <= 7u relative error (x^3, two products, one sum,
  two constants); exp(-2v) as exp2(-2v log2 e) adds |2v| u from the scaled
  argument and 2u from the hardware exp2; 1 + e, the reciprocal and the
  product add 3u, and the result moves by at most e/(1+e) <= 1 times the
  relative error of e. Bound: |dev - ref| <= (6 + 18|v|) u |ref| + (|x| + 1)
  2^-126: where 1 + e exceeds 2^126 the hardware reciprocal flushes to zero,
  so results below |x| 2^-126 (x < -10.06) come out as zero.
- softmax exponentials: Q is pre-scaled by fl(log2 e / sqrt(hs)), so each
  exponent carries <= 2u (|s| + |max|) log2 e of error, the difference to
  the running max u |s - max|, the hardware exp2 u, and the sum of T
  probabilities gamma_T; PV with one-hot values is exact. Bound:
  |p - p64| <= (8 + 3 (|s| + |max|) + T) u p64 + 2^-126.
- GEMM (float64 brute force at odd shapes): |Y - Y64| <= gamma_{K+4}
  (sum_k |x_k w_k| + |b| + |Y_old|), the textbook bound for a sum in any
  order plus the epilogue's roundings.
- LayerNorm: |dev - ref| <= gamma_{2C+32} (|w| r (|x| + |mean|) + |b|).
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
TINY = 2.0 ** -126
LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat", "libcngpt_kat.so")
_F = ctypes.POINTER(ctypes.c_float)


@pytest.fixture(scope="module")
def kat():
    assert os.path.exists(LIB), "tests/kat/libcngpt_kat.so not built (run __graft_entry__.build())"
    lib = ctypes.CDLL(LIB)
    lib.kat_error.restype = ctypes.c_char_p
    for name in ("kat_gemm", "kat_gemm_ln", "kat_layernorm", "kat_attention", "kat_attention_row"):
        getattr(lib, name).restype = ctypes.c_int
    return lib


def fp(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def check(lib, rc):
    assert rc == 0, lib.kat_error().decode()


def gemm(lib, X, W, b, M, N, K, epi, path, Y=None):
    Y = np.zeros((M, N), np.float32) if Y is None else Y.copy()
    check(lib, lib.kat_gemm(fp(X), fp(W), fp(b), fp(Y), M, N, K, epi, path))
    return Y


# ------------------------------------------------------------------ known answers

# (path, M): decode product; weight-streaming product; MFMA tiles
LINEAR_PATHS = [(1, 2), (0, 2), (0, 130)]


@pytest.mark.parametrize("K", [4, 16, 32])
@pytest.mark.parametrize("path,M", LINEAR_PATHS)
def test_linear_known_answer(kat, path, M, K):
    """check_ops.c:69-82: X = I, W = [[2, 3], [4, 5]], b = [1, -1] ->
    [[3, 3], [4, 4]] within 1e-5."""
    rng = np.random.default_rng(M + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    X[:2] = 0
    X[0, 0] = X[1, 1] = 1
    W = np.zeros((2, K), np.float32)
    W[:, :2] = [[2, 3], [4, 5]]
    b = np.array([1, -1], np.float32)
    Y = gemm(kat, X, W, b, M, 2, K, 1, path)
    assert np.abs(Y[:2] - np.array([[3, 3], [4, 4]], np.float32)).max() <= 1e-5, Y[:2]


def test_layernorm_known_answer(kat):
    """check_ops.c:118-136: LayerNorm([1, 2, 3, 4]) with w = 1, b = 0."""
    x = np.array([[1, 2, 3, 4]], np.float32)
    out = np.zeros_like(x)
    check(kat, kat.kat_layernorm(fp(x), fp(np.ones(4, np.float32)),
                                 fp(np.zeros(4, np.float32)), fp(out), 1, 4))
    want = np.array([-1.3416, -0.4472, 0.4472, 1.3416])
    assert np.abs(out[0] - want).max() <= 1e-3, out
    assert abs(float(out.sum())) <= 1e-4


def gelu_through(kat, x, path):
    """GELU of each x through the bias+GELU epilogue: rows [x, 0, 0, 0]
    times the weight row [1, 0, 0, 0], bias 0."""
    M = x.size
    X = np.zeros((M, 4), np.float32)
    X[:, 0] = x
    W = np.array([[1, 0, 0, 0]], np.float32)
    return gemm(kat, X, W, np.zeros(1, np.float32), M, 1, 4, 2, path)[:, 0]


@pytest.mark.parametrize("path,M", [(1, 4), (0, 4), (0, 130)])
def test_gelu_known_answer(kat, path, M):
    """check_ops.c:146-157: gelu(0) = 0 (1e-4), gelu(1) = 0.8413,
    gelu(-1) = -0.1587, gelu(2) = 1.9545 (1e-3)."""
    x = np.zeros(M, np.float32)
    x[:4] = [0, 1, -1, 2]
    g = gelu_through(kat, x, path)
    assert abs(g[0]) <= 1e-4
    assert np.abs(g[1:4] - np.array([0.8413, -0.1587, 1.9545])).max() <= 1e-3, g[:4]


def one_hot_attention(scores_rows, hs=64):
    """qkv [B, T, 3C] (C = hs, one head) whose final query row attends with
    the given scores: q = [sqrt(hs), 0, ...], k_j = [s_j, 0, ...] (so
    q.k_j / sqrt(hs) = s_j exactly), v_j = e_j (so output element j is the
    probability of key j)."""
    B, T = scores_rows.shape
    assert T <= hs
    qkv = np.zeros((B, T, 3 * hs), np.float32)
    qkv[:, T - 1, 0] = np.sqrt(hs)
    qkv[:, :, hs] = scores_rows
    qkv[:, np.arange(T), 2 * hs + np.arange(T)] = 1.0
    return qkv


def attention_probs(kat, scores, kind):
    B, T = scores.shape
    hs = 64
    qkv = one_hot_attention(scores.astype(np.float32), hs)
    if kind == "causal":
        out = np.zeros((B, T, hs), np.float32)
        check(kat, kat.kat_attention(fp(qkv), fp(out), B, T, hs, 1))
        return out[:, T - 1, :T]
    out = np.zeros((B, hs), np.float32)
    check(kat, kat.kat_attention_row(fp(qkv), fp(out), B, T, hs, 1))
    return out[:, :T]


@pytest.mark.parametrize("kind", ["causal", "row"])
def test_softmax_known_answer(kat, kind):
    """check_ops.c:165-182: softmax([1, 2, 3]) = [0.0900, 0.2447, 0.6652]
    (1e-3), rows sum to 1 (1e-5); softmax([100, 100, 100]) = 1/3 (1e-5)."""
    p = attention_probs(kat, np.array([[1, 2, 3], [100, 100, 100]], np.float32), kind)
    assert np.abs(p[0] - np.array([0.0900, 0.2447, 0.6652])).max() <= 1e-3, p[0]
    assert abs(float(p[0].sum()) - 1) <= 1e-5
    assert np.abs(p[1] - 1 / 3).max() <= 1e-5, p[1]


# ------------------------------------------------------------------ error bounds

def gelu64(x):
    """0.5 x (1 + tanh v) in float64 as x expit(2v) (1 + tanh v = 2 expit(2v)
    exactly; scipy's expit keeps full relative precision where float64's
    1 + tanh(v) cancels to zero, v < -19)."""
    from scipy.special import expit
    x = x.astype(np.float64)
    v = np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)
    return x * expit(2 * v), v


@pytest.mark.parametrize("path", [0, 1])
def test_gelu_error_bound_dense_grid(kat, path):
    """Device GELU vs float64 on 48001 points over [-12, 12] (step 5e-4) and
    the saturation ends +-20, +-50, +-1e3, +-1e4, within (6 + 18|v|) u |ref|
    + (|x| + 1) 2^-126. path 0: the MFMA tiles' epilogue; path 1: the
    decode product's (in batches of 8 rows)."""
    x = np.concatenate([np.linspace(-12, 12, 48001),
                        [-1e4, -1e3, -50, -20, 20, 50, 1e3, 1e4]]).astype(np.float32)
    if path == 0:
        g = gelu_through(kat, x, 0)
    else:
        g = np.concatenate([gelu_through(kat, x[i:i + 8], 1) for i in range(0, x.size, 8)])
    ref, v = gelu64(x)
    assert np.isfinite(g).all()
    err = np.abs(g.astype(np.float64) - ref)
    bound = (6 + 18 * np.abs(v)) * U * np.abs(ref) + (np.abs(x) + 1) * TINY
    worst = int(np.argmax(err / bound))
    print(f"gelu path {path}: max rel err {float((err / np.maximum(np.abs(ref), TINY)).max()):.3e}"
          f", worst err/bound {float(err[worst] / bound[worst]):.3f} at x={x[worst]}", flush=True)
    assert np.all(err <= bound), (x[worst], g[worst], ref[worst])
    # the saturation ends are exact: x for large x, zero for large -x
    assert np.all(g[x >= 20] == x[x >= 20]) and np.all(g[x <= -50] == 0)


@pytest.mark.parametrize("kind", ["causal", "row"])
def test_softmax_error_bound_dense_grid(kat, kind):
    """Probabilities of 64 sequences x 64 keys whose scores are a shuffled
    grid of 4096 points over [-12, 12] (exponents down to -24), plus rows at
    the saturation ends (score gaps of 50 and 100, where e^-100 is below
    fp32's normal range), vs float64 softmax of the same fp32 scores, within
    (8 + 3 (|s| + |max|) + T) u p64 + 2^-126."""
    rng = np.random.default_rng(17)
    grid = np.linspace(-12, 12, 4096).astype(np.float32)
    S = rng.permutation(grid).reshape(64, 64)
    sat = np.zeros((2, 64), np.float32)
    sat[0, :3] = [50, -50, 0]
    sat[0, 3:] = -40
    sat[1, :] = 100
    sat[1, 1::2] = 0
    S = np.concatenate([S, sat])
    p = attention_probs(kat, S, kind).astype(np.float64)
    s64 = S.astype(np.float64)
    mx = s64.max(1, keepdims=True)
    e = np.exp(s64 - mx)
    ref = e / e.sum(1, keepdims=True)
    bound = (8 + 3 * (np.abs(s64) + np.abs(mx)) + 64) * U * ref + TINY
    err = np.abs(p - ref)
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    print(f"softmax {kind}: max err/bound {float((err / bound).max()):.3f} at {worst}", flush=True)
    assert np.all(err <= bound), (worst, p[worst], ref[worst])
    assert np.abs(p.sum(1) - 1).max() <= 64 * U


@pytest.mark.parametrize("path,M,N,K,epi", [
    (0, 130, 81, 1600, 1),    # MFMA tiles, ragged edges, K = 1600 (XL)
    (0, 200, 333, 36, 2),     # register-staged tiles (K not a multiple of 16), GELU
    (0, 257, 129, 768, 3),    # direct-to-LDS BK = 32, residual
    (0, 128, 2304, 768, 1),   # 32 x 48 tiles over M = 128 rows (k_rows), no K split
    (0, 100, 3072, 768, 2),   # 32 x 48 tiles, ragged rows, GELU
    (0, 128, 768, 3072, 3),   # 32 x 48 tiles with K split 4 ways, residual reduce
    (0, 97, 1000, 1600, 3),   # 32 x 64 tiles, ragged rows and columns, K = 1600 split, residual
    (0, 128, 50, 64, 2),      # 32 x 32 tiles, one 64-k stage, ragged columns, GELU
    (0, 128, 4096, 1024, 2),  # 32 x 64 tiles, 256 of them, GELU
    (0, 120, 1024, 4096, 3),  # 32 x 64 tiles with K split 4 ways, ragged rows, residual
    (0, 256, 771, 768, 3),    # two row tiles, ragged columns, K split
    (0, 65, 50, 36, 1),       # register-staged tiles, K = 36, one tile
    (0, 300, 200, 48, 1),     # whole 128 x 128 tiles at BK = 16 (K = 48: three steps)
    (0, 2000, 1000, 80, 3),   # whole tiles at BK = 16, K = 80, residual
    (0, 4100, 1100, 112, 2),  # whole tiles at BK = 16 over more than 256 tiles, GELU
    (0, 2048, 768, 768, 3),   # 64 x 48 tiles, two per CU (M = 2048), residual
    (0, 2048, 768, 3072, 3),  # 64 x 48 tiles over K = 3072, residual
    (0, 2048, 3072, 768, 2),  # 64 x 96 tiles, two rounds at two per CU, GELU
    (0, 1000, 2304, 768, 1),  # 64 x 96 tiles, ragged rows
    (0, 4096, 2304, 768, 1),  # 64 x 96 tiles, three rounds at two per CU
    (0, 1024, 768, 768, 3),   # 128 x 128 tiles with K split (M = 1024), residual reduce
    (0, 2048, 2304, 768, 1),  # 128 x 144 tiles, one per CU
    (0, 1100, 4000, 1600, 3), # stream-K: 9 x 32 ragged tiles, residual
    (0, 1280, 7680, 256, 3),  # 600 tiles over 256 workgroups: a whole-tile round, then stream-K
    (0, 1000, 19400, 64, 2),  # 8 x 152 ragged tiles over 512 workgroups: whole-tile round, GELU
    (0, 37, 100, 3072, 3),    # 37 rows: 32 x 32 tiles (k_rows), a one-tile-wide K split, residual
    (0, 33, 768, 768, 3),     # 33 rows: a second row tile of one row, K split, residual
    (0, 64, 2304, 768, 1),    # 64 rows: two row tiles of k_rows
    (0, 37, 100, 3040, 3),    # 37 rows, K not a multiple of 64: weight-streaming, split over K
    (0, 5, 2304, 768, 1),     # weight-streaming, QKV width
    (0, 8, 3072, 1024, 1),    # weight-streaming, four wavefronts per column block, no K split
    (0, 13, 4100, 1000, 2),   # two phases per block, ragged columns and K, GELU
    (0, 30, 6400, 1600, 3),   # two phases per block at 30 rows, residual
    (0, 16, 3200, 36, 1),     # four phases per block, K = 36 (one step, three phases empty)
    (2, 8, 4096, 1024, 2),    # packed weights, four phases per block
    (2, 37, 100, 3040, 3),    # weight-streaming from packed weights, split over K
    (2, 20, 771, 1600, 2),    # packed weights, ragged last column block, GELU
    (2, 100, 333, 36, 1),     # packed, K = 36 (zero-padded last step), 128-row tiles
    (2, 128, 2304, 768, 1),   # 128 rows: 32 x 48 tiles (the packed copy unused)
    (1, 2, 771, 1024, 3),     # decode product
])
def test_gemm_error_bound_float64(kat, path, M, N, K, epi):
    """Every product variant vs a float64 product at odd shapes, within the
    gamma_{K+4} bound (the reference pins its GEMM only by the 2x2 KAT;
    this pins realistic shapes)."""
    rng = np.random.default_rng(M * N + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    Y0 = rng.standard_normal((M, N)).astype(np.float32)
    Y = gemm(kat, X, W, b, M, N, K, epi, path, Y0)
    acc = X.astype(np.float64) @ W.astype(np.float64).T
    mag = np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64)).T + np.abs(b)
    gelu_err = 0.0
    if epi == 1:
        ref = acc + b
    elif epi == 2:
        # an input error d moves GELU by at most 1.13 d (its slope stays in
        # [-0.13, 1.13]); GELU's own rounding as in the dense-grid bound
        ref, v = gelu64(acc + b)
        mag = 1.13 * mag
        gelu_err = (6 + 18 * np.abs(v)) * U * np.abs(ref) + (np.abs(acc + b) + 1) * TINY
    else:
        ref = (Y0 + acc) + b
        mag = mag + np.abs(Y0)
    bound = (K + 4) * U * mag + gelu_err + TINY
    err = np.abs(Y - ref)
    print(f"gemm path {path} {M}x{N}x{K} epi {epi}: max err/bound "
          f"{float((err / bound).max()):.3f}", flush=True)
    assert np.all(err <= bound)


@pytest.mark.parametrize("M,N,K,epi", [
    (3, 2304, 768, 1), (24, 3200, 800, 2), (40, 1600, 6432, 3), (64, 50257, 96, 0),
    (100, 333, 36, 3), (128, 771, 1280, 1), (8, 3072, 1024, 1), (32, 6400, 1600, 2),
])
def test_gemm_packed_weights_bitwise(kat, M, N, K, epi):
    """The packed copy of W only moves where each weight is read from: the
    few-row product gives bit-identical results from it and from W."""
    rng = np.random.default_rng(7 * M + N + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    Y0 = rng.standard_normal((M, N)).astype(np.float32)
    Yr = gemm(kat, X, W, b, M, N, K, epi, 0, Y0.copy())
    Yp = gemm(kat, X, W, b, M, N, K, epi, 2, Y0.copy())
    assert np.isfinite(Yr).all()
    assert np.array_equal(Yr.view(np.uint32), Yp.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [
    (8, 1024, 1024), (32, 1600, 6400), (5, 1280, 5120), (40, 768, 3072), (64, 2048, 2048),
    (17, 1600, 1600), (128, 768, 3072),
])
def test_gemm_layernorm_in_split_sum(kat, M, N, K):
    """The residual product whose split sum also forms the next LayerNorm
    (the sum launch over whole rows): the residual stream within the float64
    error bound, and the LayerNorm within 1e-5 of a float64 LayerNorm of the
    float32 rows."""
    check_gemm_layernorm(kat, M, N, K, split=True)


@pytest.mark.parametrize("M,N,K", [(2048, 768, 3072), (2048, 768, 768)])
def test_gemm_layernorm_after_whole_k(kat, M, N, K):
    """The same product and LayerNorm where the product runs whole K (64 x 48
    tiles at 2048 rows) and the LayerNorm is a launch of its own."""
    check_gemm_layernorm(kat, M, N, K, split=False)


def check_gemm_layernorm(kat, M, N, K, split):
    rng = np.random.default_rng(13 * M + N + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    Y0 = rng.standard_normal((M, N)).astype(np.float32)
    lw = (1 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    lb = (0.1 * rng.standard_normal(N)).astype(np.float32)
    Y = Y0.copy()
    ln = np.zeros((M, N), np.float32)
    splits = kat.kat_gemm_ln(fp(X), fp(W), fp(b), fp(Y), fp(lw), fp(lb), fp(ln), M, N, K)
    assert splits > 0, kat.kat_error().decode()
    assert (splits > 1) == split, splits
    acc = X.astype(np.float64) @ W.astype(np.float64).T
    mag = np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64)).T + np.abs(b) + np.abs(Y0)
    assert np.all(np.abs(Y - ((Y0 + acc) + b)) <= (K + 4) * U * mag + TINY)
    y = Y.astype(np.float64)
    mu = y.mean(1, keepdims=True)
    ref = (y - mu) / np.sqrt(((y - mu) ** 2).mean(1, keepdims=True) + 1e-5) * lw + lb
    assert np.abs(ln - ref).max() < 1e-5


@pytest.mark.parametrize("C", [4, 64, 768, 1024, 1600])
def test_layernorm_error_bound_float64(kat, C):
    rng = np.random.default_rng(C)
    rows = 257
    x = (rng.standard_normal((rows, C)) * 3 + rng.standard_normal((rows, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.05 * rng.standard_normal(C)).astype(np.float32)
    out = np.zeros_like(x)
    check(kat, kat.kat_layernorm(fp(x), fp(w), fp(b), fp(out), rows, C))
    x64 = x.astype(np.float64)
    m = x64.mean(1, keepdims=True)
    r = 1 / np.sqrt(((x64 - m) ** 2).mean(1, keepdims=True) + 1e-5)
    ref = (x64 - m) * r * w + b
    bound = (2 * C + 32) * U * (np.abs(w) * r * (np.abs(x64) + np.abs(m)) + np.abs(b)) + TINY
    err = np.abs(out - ref)
    print(f"layernorm C={C}: max err/bound {float((err / bound).max()):.3f}", flush=True)
    assert np.all(err <= bound)
