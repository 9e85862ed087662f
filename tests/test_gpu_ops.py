"""Per-op parity of the HIP kernels (through the C ABI) against the oracle.

Bar: bit-exact.  Integer block dots are exact by construction, and every
f32 step reproduces the reference's operation order, so outputs must match
the oracle to the last bit (compared as uint32 patterns).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits(a, b):
    a, b = np.asarray(a, np.float32).ravel(), np.asarray(b, np.float32).ravel()
    bad = np.nonzero(bits(a) != bits(b))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:5]}: {a[bad[:5]]} vs {b[bad[:5]]}"


def test_math_primitives(gpu, oracle):
    from yallma3_mini_inference_amd import ops
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-104, 88.7, 60000), rng.uniform(-12, 12, 5536),
                        np.array([0.0, 1.0, -1.0, 1e-30, 3.0e38, -87.4, -103.5])]).astype(np.float32)
    e, s, r, h = ops.math_selftest(x)
    assert_bits(e, [oracle.expf(float(v)) for v in x])
    assert_bits(s, np.sqrt(np.abs(x)))               # correctly rounded sqrt
    with np.errstate(divide="ignore"):
        assert_bits(r, np.float32(1.0) / x)          # correctly rounded division
    idx = (np.arange(x.size) & 0xFFFF).astype(np.uint16)
    ref = idx.view(np.float16).astype(np.float32)
    ok = (bits(h) == bits(ref)) | (np.isnan(h) & np.isnan(ref))
    assert ok.all()


@pytest.mark.parametrize("fmt", [0, 1])
def test_quantize(gpu, oracle, fmt):
    from yallma3_mini_inference_amd import WeightFormat, quantize
    rng = np.random.default_rng(1 + fmt)
    x = rng.normal(0, 1, 32 * 300).astype(np.float32)
    x[64:96] = 0.0
    x[96:128] = np.linspace(-3.5, 3.5, 32)
    q, s = quantize(WeightFormat(fmt), x)
    oq, os_ = oracle.quantize(fmt, x)
    np.testing.assert_array_equal(q, oq)
    assert_bits(s, os_)


def _near_tie_groups(rng, n_groups, qmax):
    """Groups whose values sit on or within a few ulps of x/scale = k + 1/2.

    Each group holds its absmax (fixing scale = absmax/qmax) and 31 values
    built from (k + 0.5) * scale, nudged by -3..3 ulps, so both rounding
    directions of the reference's quotient are exercised."""
    out = []
    for _ in range(n_groups):
        am = np.float32(rng.uniform(0.05, 900.0))
        sc = np.float32(am / np.float32(qmax))
        k = rng.integers(-qmax, qmax, 31)
        v = ((k + 0.5) * np.float64(sc)).astype(np.float32)
        for i, u in enumerate(rng.integers(-3, 4, 31)):
            for _ in range(abs(int(u))):
                v[i] = np.nextafter(v[i], np.float32(np.inf if u > 0 else -np.inf))
        v = np.clip(v, -am, am)
        out.append(np.concatenate([[am if rng.random() < 0.5 else -am], v]).astype(np.float32))
    return np.concatenate(out)


@pytest.mark.parametrize("fmt", [0, 1])
def test_quantize_ties(gpu, oracle, fmt):
    # The GPU quantizer divides only near half-integer quotients; this
    # drives many values onto and around those boundaries, plus power-of-two
    # scales (exact ties), subnormal scales, NaN and infinities.
    from yallma3_mini_inference_amd import WeightFormat, quantize
    qmax = 127 if fmt == 0 else 7
    rng = np.random.default_rng(11 + fmt)
    parts = [_near_tie_groups(rng, 400, qmax)]
    exact = np.concatenate([[float(qmax)], (np.arange(31) % (2 * qmax) - qmax) + 0.5]).astype(np.float32)
    parts.append(exact)                                   # scale 1: every quotient an exact tie
    parts.append(exact * np.float32(2.0 ** -20))          # power-of-two scale
    parts.append((rng.normal(0, 1, 32) * 1e-41).astype(np.float32))   # subnormal scale
    nan = rng.normal(0, 1, 32).astype(np.float32)
    nan[5] = np.nan
    parts.append(nan)
    inf = rng.normal(0, 1, 32).astype(np.float32)
    inf[9] = np.inf
    parts.append(inf)
    x = np.concatenate(parts)
    with np.errstate(invalid="ignore", over="ignore"):
        q, s = quantize(WeightFormat(fmt), x)
        oq, os_ = oracle.quantize(fmt, x)
    np.testing.assert_array_equal(q, oq)
    assert_bits(s, os_)


def test_matmul_reference_kat(gpu):
    # tests/matmul_q8_tests.rs:30-53 through the HIP GEMV
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, matmul
    n, o = 64, 33
    w = QuantizedWeight.upload(WeightFormat.Q8_0, np.ones(o * n, np.int8), np.ones(o * n // 32, np.float32), o, n)
    out = np.zeros(o, np.float32)
    matmul(out, np.ones(n, np.int8), np.ones(n // 32, np.float32), w, n, o)
    assert np.all(np.abs(out - n) < 1e-5)


def _gguf_q8_blocks(wf):
    """GGUF Q8_0 blocks of a float matrix (d = absmax/127 as f16, q = round(x/d))."""
    blocks = wf.reshape(-1, 32)
    amax = np.abs(blocks).max(axis=1)
    d = (amax / 127.0).astype(np.float32)
    inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.round(blocks * inv[:, None]).astype(np.int8)
    out = np.zeros((blocks.shape[0], 34), np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel(), q.ravel(), d.astype(np.float16).astype(np.float32)


# 128-512 blocks per row, at most 2048 rows and 2048 x 256 row-blocks take
# one wavefront per row: whole slots, a partial slot (160 blocks), 512
# blocks, both bounds met exactly (2048 x 256, 1024 x 512), and one past each
# on the 16-lane rows
@pytest.mark.parametrize("batch,n,o", [(1, 2048, 2048), (1, 8192, 1024), (3, 576, 190), (2, 4096, 37),
                                       (1, 14336, 128), (1, 5120, 77), (2, 16384, 64), (1, 8192, 2048),
                                       (1, 8192, 2049), (1, 16384, 1024), (1, 16384, 1025)])
def test_matmul_q8_parity(gpu, oracle, batch, n, o):
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, matmul
    rng = np.random.default_rng(n + o)
    wf = rng.normal(0, 0.02, o * n).astype(np.float32)
    blk, wq, ws = _gguf_q8_blocks(wf)
    w = QuantizedWeight.upload_gguf(WeightFormat.Q8_0, blk, o, n)
    xq, xs = oracle.quantize(0, rng.normal(0, 1, batch * n).astype(np.float32))
    init = rng.normal(0, 1, batch * o).astype(np.float32)     # `+=` columns keep it, tail columns drop it
    out = matmul(init.copy(), xq, xs, w, n, o)
    ref = oracle.matmul_q8_slices(init.copy(), xq, xs, wq, ws, n, o)
    assert_bits(out, ref)


@pytest.mark.parametrize("batch,n,o", [(1, 2048, 512), (2, 8192, 256), (1, 576, 36), (1, 14336, 256),
                                       (1, 5120, 40)])
def test_matmul_q4_parity(gpu, oracle, batch, n, o):
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, matmul
    rng = np.random.default_rng(7 * n + o)
    wq = rng.integers(0, 16, o * n).astype(np.int8)            # reference Q4_0: unsigned nibbles
    ws = (rng.normal(0, 0.003, o * n // 32)).astype(np.float16).astype(np.float32)
    w = QuantizedWeight.upload(WeightFormat.Q4_0, wq, ws, o, n)
    xq, xs = oracle.quantize(1, rng.normal(0, 1, batch * n).astype(np.float32))
    out = matmul(np.zeros(batch * o, np.float32), xq, xs, w, n, o)
    ref = oracle.matmul_q8_slices(np.zeros(batch * o, np.float32), xq, xs, wq, ws, n, o)
    assert_bits(out, ref)


@pytest.mark.parametrize("fmt,batch,n,o", [(0, 16, 2048, 256), (0, 130, 576, 190), (0, 257, 8192, 128),
                                           (1, 64, 2048, 384), (1, 200, 1536, 96), (1, 256, 14336, 512),
                                           (0, 96, 14336, 136)])
def test_matmul_mfma_parity(gpu, oracle, fmt, batch, n, o):
    # batches of >= 16 rows run the int8-MFMA GEMM: partial token and row
    # tiles, the `+=` columns and the `=` tail columns, both formats
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, matmul
    rng = np.random.default_rng(11 * n + o + batch)
    if fmt == 0:
        wf = rng.normal(0, 0.02, o * n).astype(np.float32)
        blk, wq, ws = _gguf_q8_blocks(wf)
        w = QuantizedWeight.upload_gguf(WeightFormat.Q8_0, blk, o, n)
    else:
        wq = rng.integers(0, 16, o * n).astype(np.int8)
        ws = (rng.normal(0, 0.003, o * n // 32)).astype(np.float16).astype(np.float32)
        w = QuantizedWeight.upload(WeightFormat.Q4_0, wq, ws, o, n)
    xq, xs = oracle.quantize(fmt, rng.normal(0, 1, batch * n).astype(np.float32))
    init = rng.normal(0, 1, batch * o).astype(np.float32)
    out = matmul(init.copy(), xq, xs, w, n, o, fmt=WeightFormat(fmt))
    ref = oracle.matmul_q8_slices(init.copy(), xq, xs, wq, ws, n, o)
    assert_bits(out, ref)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("negz", [False, True])
@pytest.mark.parametrize("batch,n,o", [(96, 512, 384), (2048, 256, 2304)])
def test_matmul_mfma_special_scales(gpu, oracle, fmt, negz, batch, n, o):
    # The GEMM folds the int32-to-f32 convert into an FMA on a biased dot for
    # f16 scales.  That form differs from the reference's only in the sign of
    # a zero term, which the sum can show only from a -0 start, and on
    # non-finite scales; both must take the reference's form.  Rows 0..127:
    # zero, -0, negative, smallest-subnormal and largest f16 scales; token 10
    # has all-zero activations (every term of its outputs is a signed zero),
    # token 11 two zero blocks.  Initial values are +0 there (the biased form
    # stays exact) or -0 (negz: the workgroup must fall back).  Rows 128..255
    # hold inf, -inf and NaN scales.  (96, 512, 384) runs 64-token tiles,
    # (2048, 256, 2304) 128-token tiles.
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, matmul
    rng = np.random.default_rng(5 + fmt + 2 * negz + n)
    nb = n // 32
    if fmt == 0:
        wq = rng.integers(-128, 128, o * n).astype(np.int8)
    else:
        wq = rng.integers(0, 16, o * n).astype(np.int8)
    ws = rng.normal(0, 0.003, (o, nb)).astype(np.float16).astype(np.float32)
    ws[3, :] = 0.0
    ws[4, :] = -0.0
    ws[5, 2] = 0.0
    ws[6, :] = -np.abs(ws[6, :])
    ws[7, 0] = np.float32(2.0 ** -24)
    ws[8, 1] = np.float32(65504.0)
    ws[9, :] = -np.float32(2.0 ** -24)
    ws[130, 3] = np.inf
    ws[131, 5] = -np.inf
    ws[132, 1] = np.nan
    w = QuantizedWeight.upload(WeightFormat.Q8_0 if fmt == 0 else WeightFormat.Q4_0, wq, ws.ravel(), o, n)
    x = rng.normal(0, 1, (batch, n)).astype(np.float32)
    x[10, :] = 0.0
    x[11, :64] = 0.0
    xq, xs = oracle.quantize(fmt, x.ravel())
    init = rng.normal(0, 1, (batch, o)).astype(np.float32)
    init[10, :128] = -0.0 if negz else 0.0
    init[11, :16] = -0.0 if negz else 0.0
    out = matmul(init.ravel().copy(), xq, xs, w, n, o, fmt=WeightFormat(fmt))
    with np.errstate(invalid="ignore", over="ignore"):
        ref = oracle.matmul_q8_slices(init.ravel().copy(), xq, xs, wq, ws.ravel(), n, o)
    nan = np.isnan(ref)
    assert nan.any() and np.array_equal(np.isnan(out), nan)
    assert_bits(np.where(nan, 0, out), np.where(nan, 0, ref))
    zero_rows = ref.reshape(batch, o)[10, :128]
    assert (np.signbit(zero_rows).any() if negz else True) and np.all(zero_rows == 0)


def test_matmul_format_mismatch_raises(gpu):
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, YlError, matmul
    w = QuantizedWeight.upload(WeightFormat.Q8_0, np.ones(64, np.int8), np.ones(2, np.float32), 2, 32)
    with pytest.raises(YlError):
        matmul(np.zeros(2, np.float32), np.ones(32, np.int8), np.ones(1, np.float32), w, 32, 2,
               fmt=WeightFormat.Q4_0)


def test_matmul_isolated_8192x2048(gpu, oracle):
    # the isolated Q8_0 matvec workload: W 8192x2048 ~N(0,0.02) GGUF Q8_0, x ~N(0,1) Q8_0, seed 0
    from yallma3_mini_inference_amd import QuantizedWeight, WeightFormat, matmul
    from yallma3_mini_inference_amd.synth import ModelConfig  # noqa: F401  (same generator family)
    import ctypes as C
    o, n = 8192, 2048
    wf = np.zeros(o * n, np.float32)
    xf = np.zeros(n, np.float32)
    gpu.lib().yl_synthetic_normal(0, 0, 0, wf.size, C.c_float(0.02), wf.ctypes.data)
    gpu.lib().yl_synthetic_normal(0, 1, 0, xf.size, C.c_float(1.0), xf.ctypes.data)
    blk, wq, ws = _gguf_q8_blocks(wf)
    w = QuantizedWeight.upload_gguf(WeightFormat.Q8_0, blk, o, n)
    xq, xs = oracle.quantize(0, xf)
    out = matmul(np.zeros(o, np.float32), xq, xs, w, n, o)
    ref = oracle.matmul_q8_slices(np.zeros(o, np.float32), xq, xs, wq, ws, n, o)
    assert_bits(out, ref)


@pytest.mark.parametrize("size,batch,qfmt", [(2048, 1, 0), (576, 3, 0), (4096, 2, 1), (104, 1, -1), (2048, 1, -1)])
def test_rmsnorm_quantize(gpu, oracle, size, batch, qfmt):
    from yallma3_mini_inference_amd import ops
    rng = np.random.default_rng(size + batch)
    x = rng.normal(0, 2, (batch, size)).astype(np.float32)
    w = rng.normal(1, 0.2, size).astype(np.float32)
    xn, q, s = ops.rmsnorm_quantize(x, w, 1e-5, qfmt)
    ref = np.stack([oracle.rmsnorm(x[t], w, 1e-5) for t in range(batch)])
    assert_bits(xn, ref)
    if qfmt >= 0:
        oq, os_ = oracle.quantize(qfmt, ref.ravel())
        np.testing.assert_array_equal(q, oq)
        assert_bits(s, os_)


@pytest.mark.parametrize("hd,nh,nkv,theta,pos,batch", [(64, 32, 8, 500000.0, 0, 1), (64, 9, 3, 10000.0, 377, 2),
                                                       (128, 32, 8, 500000.0, 8300, 3)])
def test_rope(gpu, oracle, hd, nh, nkv, theta, pos, batch):
    from yallma3_mini_inference_amd import ops
    from yallma3_mini_inference_amd._lib import RopeParams
    rng = np.random.default_rng(pos)
    q = rng.normal(0, 1, (batch, nh * hd)).astype(np.float32)
    k = rng.normal(0, 1, (batch, nkv * hd)).astype(np.float32)
    p = RopeParams(hd, nh, nkv, theta, 1.0, 0.0, 1.0, 8192)
    gq, gk = ops.rope_gguf(p, q, k, pos, batch)
    op = oracle.rope_params(hd, nh, nkv, theta, original_ctx_len=8192)
    for t in range(batch):
        rq, rk = q[t].copy(), k[t].copy()
        oracle.rope_gguf(op, rq, rk, pos + t)
        assert_bits(gq[t], rq)
        assert_bits(gk[t], rk)


@pytest.mark.parametrize("hd,nh,nkv,theta,fs,ext,attn,orig,pos,batch", [
    (64, 32, 8, 500000.0, 0.25, 1.0, 1.1, 1024, 0, 1), (64, 4, 2, 10000.0, 0.25, 1.0, 1.1, 1024, 3001, 3),
    (64, 9, 3, 500000.0, 0.125, 0.5, 0.9, 2048, 777, 2), (128, 32, 8, 500000.0, 1 / 32, 1.0, 1.0, 8192, 8300, 2),
    (32, 8, 4, 500000.0, 0.25, 1.0, 1.2, 2048, 40, 5), (128, 8, 2, 10000.0, 0.5, 0.5, 1.05, 4096, 20000, 1)])
def test_rope_yarn(gpu, oracle, hd, nh, nkv, theta, fs, ext, attn, orig, pos, batch):
    # rope_gguf's YaRN branch (util.rs:653-724): the library's angle table and
    # rotation against the oracle's, bit for bit
    from yallma3_mini_inference_amd import ops
    from yallma3_mini_inference_amd._lib import RopeParams
    rng = np.random.default_rng(pos + hd)
    q = rng.normal(0, 1, (batch, nh * hd)).astype(np.float32)
    k = rng.normal(0, 1, (batch, nkv * hd)).astype(np.float32)
    gq, gk = ops.rope_gguf(RopeParams(hd, nh, nkv, theta, fs, ext, attn, orig), q, k, pos, batch)
    op = oracle.rope_params(hd, nh, nkv, theta, fs, ext, attn, orig)
    for t in range(batch):
        rq, rk = q[t].copy(), k[t].copy()
        oracle.rope_gguf(op, rq, rk, pos + t)
        assert_bits(gq[t], rq)
        assert_bits(gk[t], rk)


@pytest.mark.parametrize("batch,start,nh,nkv,hd", [(1, 0, 4, 2, 64), (1, 700, 32, 8, 64), (7, 13, 9, 3, 64),
                                                   (4, 250, 8, 2, 128), (1, 8447, 4, 1, 128), (1, 4999, 8, 4, 64), (1, 6000, 16, 2, 128), (1, 8191, 32, 8, 128),
                                                   (1, 3000, 9, 3, 64), (1, 2100, 2, 2, 32), (1, 5119, 8, 8, 64),
                                                   (64, 0, 4, 2, 64), (100, 37, 8, 2, 128), (130, 0, 9, 3, 64),
                                                   (70, 5, 2, 2, 32), (257, 300, 4, 1, 64)])
def test_attention(gpu, oracle, batch, start, nh, nkv, hd):
    from yallma3_mini_inference_amd import ops
    rng = np.random.default_rng(batch * 1000 + start)
    seq = start + batch
    q = rng.normal(0, 1, batch * nh * hd).astype(np.float32)
    kc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
    vc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    out = ops.attention(q, kc, vc, batch, start, nh, nkv, hd, scale)
    ref = oracle.fused_attention(q, kc, vc, seq, batch, nh, nkv, hd, start, nkv * hd, scale)
    assert_bits(out, ref)


# One-token contexts around the register P.V chains' bounds: 1 to 7 registers
# of 16 chunks (8 positions each), partial registers, a seq % 8 tail or none,
# 112 chunks (the most held in registers) and the LDS-tile chains past it.
@pytest.mark.parametrize("seq,nh,nkv,hd", [(s, 8, 2, 64) for s in (8, 9, 16, 17, 127, 128, 129, 255, 256, 257, 383,
                                                                    600, 768, 769, 775, 776, 895, 896, 897, 903, 904,
                                                                    905, 1024)]
                         + [(300, 4, 1, 128), (896, 4, 1, 128), (904, 4, 1, 128), (200, 2, 2, 32), (897, 2, 2, 32)])
def test_attention_decode_chain_lengths(gpu, oracle, seq, nh, nkv, hd):
    from yallma3_mini_inference_amd import ops
    rng = np.random.default_rng(seq * 7 + hd)
    q = rng.normal(0, 1, nh * hd).astype(np.float32)
    kc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
    vc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    out = ops.attention(q, kc, vc, 1, seq - 1, nh, nkv, hd, scale)
    ref = oracle.fused_attention(q, kc, vc, seq, 1, nh, nkv, hd, seq - 1, nkv * hd, scale)
    assert_bits(out, ref)


def test_prompt_attention_nonfinite_v(gpu, oracle):
    # an infinity in V past some rows' causal bound: the reference still adds
    # p * v there (p = 0), so those rows turn NaN; the tiled kernel must not
    # skip the masked positions then
    from yallma3_mini_inference_amd import ops
    batch, start, nh, nkv, hd = 96, 10, 4, 2, 64
    rng = np.random.default_rng(96)
    seq = start + batch
    q = rng.normal(0, 1, batch * nh * hd).astype(np.float32)
    kc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
    vc = rng.normal(0, 1, seq * nkv * hd).astype(np.float32)
    vc[(start + 80) * nkv * hd + 3] = np.inf
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    out = ops.attention(q, kc, vc, batch, start, nh, nkv, hd, scale)
    ref = oracle.fused_attention(q, kc, vc, seq, batch, nh, nkv, hd, start, nkv * hd, scale)
    nan = np.isnan(ref)
    assert nan.any() and np.array_equal(np.isnan(out), nan)
    assert_bits(out[~nan], ref[~nan])


@pytest.mark.parametrize("hidden,batch,qfmt", [(8192, 1, 0), (1536, 2, 1), (96, 1, -1)])
def test_swiglu_quantize(gpu, oracle, hidden, batch, qfmt):
    from yallma3_mini_inference_amd import ops
    rng = np.random.default_rng(hidden)
    g = rng.normal(0, 3, (batch, hidden)).astype(np.float32)
    u = rng.normal(0, 1, (batch, hidden)).astype(np.float32)
    h, q, s = ops.swiglu_quantize(g, u, qfmt)
    ref = np.stack([oracle.swiglu(g[t], u[t]) for t in range(batch)])
    assert_bits(h, ref)
    if qfmt >= 0:
        oq, os_ = oracle.quantize(qfmt, ref.ravel())
        np.testing.assert_array_equal(q, oq)
        assert_bits(s, os_)


def test_serial_sum_exact(gpu):
    # the softmax denominator's serial sum by one wavefront (forward.rs:356-361)
    import sys, os
    sys.path.insert(0, os.path.dirname(__file__))
    from serial_sum_cases import cases, sequential
    from yallma3_mini_inference_amd import ops
    segs = cases(seed=7)
    # +inf and NaN among the values (the sum stays +inf, or turns NaN)
    base = np.exp(-np.linspace(0, 4, 900)).astype(np.float32)
    for spots in ((700, np.inf), (700, np.nan), (20, np.inf), (40, np.inf, 800, np.nan)):
        w = base.copy()
        for i in range(0, len(spots), 2):
            w[spots[i]] = spots[i + 1]
        segs.append(w)
    # rows whose one-at-a-time sum drifts far from the exact sum: after a
    # first value of 1, every value is 3/4 of the sum's ulp (each add rounds
    # up by 1/4 ulp), so the segmented sum's candidate starts miss and it
    # continues one value at a time
    for n in (600, 3000):
        w = np.full(n, np.float32(0.75 * 2.0 ** -23), np.float32)
        w[0] = 1.0
        segs.append(w)
    ref = np.array([sequential(v) for v in segs], np.float32)
    nan = np.isnan(ref)
    # whole rows, and rows summed in pieces that continue from the previous
    # piece's sum (the softmax of contexts longer than LDS holds): pieces of
    # 700 (partial super-rows), 37 (inside the one-at-a-time prologue), 8192;
    # -1: the decode attention's segmented sum (candidate starts per segment);
    # -2: the long-context softmax's wide segmented sum
    for piece in (0, 700, 37, 8192, -1, -2):
        got = ops.serial_sum_selftest(segs, piece)
        assert np.array_equal(np.isnan(got), nan), piece
        assert_bits(got[~nan], ref[~nan])


def test_timed_out_wait_is_reported(gpu):
    # A GEMV whose bounded internal wait gives up marks the fault word; the
    # next synchronizing call must fail with a message and clear the word.
    from yallma3_mini_inference_amd._lib import lib, last_error, YL_OK
    L = lib()
    assert L.yl_synchronize() == YL_OK
    assert L.yl_wait_fault_selftest() == YL_OK
    st = L.yl_synchronize()
    assert st != YL_OK and "timed out" in last_error()
    assert L.yl_synchronize() == YL_OK
