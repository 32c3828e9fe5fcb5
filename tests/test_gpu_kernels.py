"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI (device pointers
allocated with torch, which is only plumbing here).

Bars: block dequant bit-exact; RoPE and residual add bit-exact; matmul/matvec within an fp32
reordering bound (the GPU reduces in a different order than the reference's sequential f32 loop);
elementwise transcendental ops within 2 ulp-scale relative error; argmax exact.
"""
import numpy as np
import pytest

import oracle as O
from inference_engine_rust_amd import engine as E
from inference_engine_rust_amd import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _stream():
    return torch.cuda.current_stream().cuda_stream


ORC = {E.Q4K: O.T_Q4K, E.Q6K: O.T_Q6K, E.Q8_0: O.T_Q8_0, E.F32: O.T_F32}
GGML = {E.Q4K: 12, E.Q6K: 14, E.Q8_0: 8}


def _rand_blocks(dt, nb, seed):
    """Random block bytes with f16 scales drawn from the full finite range (incl. subnormals)."""
    rng = np.random.default_rng(seed)
    be, bb = E.BLOCK[dt]
    b = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    h = rng.integers(0, 0x7C00, (nb, 2), dtype=np.uint16) | (rng.integers(0, 2, (nb, 2), dtype=np.uint16) << 15)
    if dt == E.Q4K:
        b[:, 0:4] = h.view(np.uint8).reshape(nb, 4)
    elif dt == E.Q6K:
        b[:, 208:210] = h[:, :1].view(np.uint8).reshape(nb, 2)
    else:
        b[:, 0:2] = h[:, :1].view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


@pytest.mark.parametrize("dt", [E.Q4K, E.Q6K, E.Q8_0])
def test_dequant_bit_exact(gpu, dt):
    nb = 4096
    blocks = _rand_blocks(dt, nb, 11 + dt)
    # a few special headers: inf / nan scales exercise the q == 0 -> 0 convention
    be, bb = E.BLOCK[dt]
    off = 208 if dt == E.Q6K else 0
    for i, bits in enumerate([0x7C00, 0xFC00, 0x7E00, 0x0001, 0x8001, 0x0000, 0x8000]):
        blocks[i * bb + off: i * bb + off + 2] = np.array([bits], np.uint16).view(np.uint8)
    want = O.dequantize(ORC[dt], blocks, nb)
    d_in = dev(blocks)
    d_out = torch.empty(nb * be, dtype=torch.float32, device="cuda")
    E.dequantize(dt, d_in.data_ptr(), nb, d_out.data_ptr(), _stream())
    got = host(d_out)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _weights(dt, k, n, seed):
    be, _ = E.BLOCK[dt] if dt != E.F32 else (1, 4)
    nel = k * n
    nb = (nel + be - 1) // be
    x = synth.normal(seed, f"w{dt}_{k}_{n}", nb * be, 0.0, 0.02)
    return x[:nel].copy() if dt == E.F32 else synth.quantize(GGML[dt], x)


def _q4k_dmin_m(w, k, n):
    """|dmin * m| of every element of a Q4_K tensor [k, n] (ggml get_scale_min_k4 min values)."""
    blocks = np.asarray(w, dtype=np.uint8).reshape(-1, 144)
    dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1)
    s = blocks[:, 4:16].astype(np.int64)
    mins = np.empty((blocks.shape[0], 8), np.float64)
    for j in range(8):
        if j < 4:
            mins[:, j] = s[:, j + 4] & 63
        else:
            mins[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    per = np.abs(dmin[:, None] * mins)  # [blocks, 8 sub-blocks of 32]
    return np.repeat(per, 32, axis=1).reshape(-1)[: k * n].reshape(n, k)


def _check_matmul(dt, k, n, m, seed=0, a=None):
    w = _weights(dt, k, n, seed)
    if a is None:
        a = synth.normal(seed + 1, f"a{k}", m * k, 0.0, 1.0).reshape(m, k)
    want = O.matmul(ORC[dt], a, w, k, n)
    dw, da = dev(w.view(np.uint8)), dev(a)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    E.matmul(da.data_ptr(), m, k, dt, dw.data_ptr(), dw.numel(), n, out.data_ptr(), _stream())
    got = host(out)
    if dt == E.F32:
        wd = w.reshape(n, k).astype(np.float64)
    else:
        be = E.BLOCK[dt][0]
        wd = O.dequantize(ORC[dt], w, (k * n + be - 1) // be)[: k * n].reshape(n, k).astype(np.float64)
    mag = np.abs(a).astype(np.float64) @ np.abs(wd).T
    if dt == E.Q4K and k % 256 == 0:
        # The decode matvec and the prefill GEMM sum d*sum(a*sc*q) and dmin*m*sum(a) separately, so
        # their reordering bound is over the magnitudes of both terms of w = d*sc*q - dmin*m.
        mag = np.abs(a).astype(np.float64) @ (np.abs(wd) + 2 * _q4k_dmin_m(w, k, n)).T
    err = np.abs(got.astype(np.float64) - want)
    # fp32 accumulation in a different order: |err| <= 2*K*eps*sum|a*w| (deterministic bound)
    bound = 2 * k * np.finfo(np.float32).eps * mag + 1e-30
    rel_bar = 1e-5
    assert np.all(err <= bound), float(np.max(err / bound))
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < rel_bar, rel


@pytest.mark.parametrize("dt,k,n", [(E.Q4K, 4096, 4096), (E.Q4K, 4096, 1024), (E.Q4K, 4096, 14336),
                                    (E.Q6K, 14336, 4096), (E.Q6K, 4096, 1000), (E.Q6K, 1408, 512),
                                    (E.Q4K, 512, 1408), (E.Q8_0, 2048, 512), (E.F32, 512, 300)])
def test_matvec_parity(gpu, dt, k, n):
    _check_matmul(dt, k, n, 1)


@pytest.mark.parametrize("dt,k,n,m", [(E.Q4K, 4096, 1024, 37), (E.Q6K, 1408, 512, 16), (E.Q6K, 14336, 256, 8),
                                      (E.Q8_0, 1024, 96, 5), (E.F32, 256, 64, 70),
                                      # matrix-core tiles: BM = 256 and 128, ragged M and N edges
                                      (E.Q4K, 4096, 2048, 300), (E.Q4K, 512, 1408, 129), (E.Q6K, 4096, 320, 256),
                                      (E.Q8_0, 2048, 200, 64), (E.F32, 1024, 136, 33)])
def test_gemm_parity(gpu, dt, k, n, m):
    _check_matmul(dt, k, n, m)


@pytest.mark.parametrize("dt,k,n", [(E.Q4K, 4096, 4096), (E.Q4K, 4096, 1024), (E.Q4K, 4096, 14336),
                                    (E.Q6K, 14336, 4096)])
def test_gemm_parity_mistral_shapes_m512(gpu, dt, k, n):
    """The four Mistral-7B projection shapes at C1's M = 512 (Q/O, K/V, gate/up, down)."""
    _check_matmul(dt, k, n, 512)


def _wide_range_rows(m, k, seed):
    """Activations over the f32 range the reference takes (src/ops/matmul.rs:176-204 multiplies any
    finite f32): row r is N(0, 1) scaled by 10^(-3 + 9 r / (m - 1)), up to 1e6; every 8th row also
    has a 32-block of same-sign values near 3000, whose per-32 sum (~1e5) exceeds fp16's 65504."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k)).astype(np.float32) * np.logspace(-3, 6, m).astype(np.float32)[:, None]
    for r in range(0, m, 8):
        b = int(rng.integers(0, k // 32))
        a[r, 32 * b:32 * b + 32] = (np.abs(rng.normal(3000.0, 100.0, 32)) * (1 if r % 16 else -1)).astype(np.float32)
    return a


@pytest.mark.parametrize("dt,k,n,m", [(E.Q4K, 4096, 1024, 512), (E.Q6K, 4096, 1024, 512), (E.Q8_0, 2048, 200, 64),
                                      (E.F32, 1024, 136, 33)])
def test_gemm_parity_full_f32_range(gpu, dt, k, n, m):
    """The op-level GEMM on activations beyond fp16's range: each row goes onto the matrix cores
    scaled by a power of two and is scaled back, so the result keeps the f32 reordering bound."""
    _check_matmul(dt, k, n, m, seed=3, a=_wide_range_rows(m, k, 40 + dt))


def test_rmsnorm_parity(gpu):
    rows, dim = 5, 4096
    x = synth.normal(1, "x", rows * dim, 0.0, 2.0).reshape(rows, dim)
    w = synth.normal(2, "w", dim, 1.0, 0.1)
    want = np.stack([O.rmsnorm(r, w, 1e-5) for r in x])
    dx, dw = dev(x), dev(w)
    out = torch.empty_like(dx)
    E.rmsnorm(dx.data_ptr(), dw.data_ptr(), rows, dim, 1e-5, out.data_ptr(), _stream())
    # The reference sums x^2 sequentially; the device sums in a tree. Both round, so the bound is
    # the summation error of a dim-term sum (dim*eps relative on sum(x^2), half that on rms).
    np.testing.assert_allclose(host(out), want, rtol=dim * np.finfo(np.float32).eps / 2 + 2e-7, atol=0)


def test_rope_bit_exact(gpu):
    nh, hd = 8, 128
    for pos in [0, 1, 513, 8191]:
        v = synth.normal(pos, "rope", nh * hd, 0.0, 1.0)
        want = np.concatenate([O.rope(v[h * hd:(h + 1) * hd], 10000.0, pos, hd, hd) for h in range(nh)])
        dv = dev(v)
        E.rope(dv.data_ptr(), nh, hd, hd, 10000.0, pos, None, _stream())
        got = host(dv)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos


def test_rope_partial_rotary_and_freq_factors(gpu):
    hd, rot = 64, 32
    v = synth.normal(3, "rp", hd, 0.0, 1.0)
    ff = np.linspace(1.0, 4.0, rot // 2).astype(np.float32)
    want = O.rope(v, 1e6, 77, hd, rot, ff=ff)
    dv = dev(v)
    E.rope(dv.data_ptr(), 1, hd, rot, 1e6, 77, ff, _stream())
    assert np.array_equal(host(dv).view(np.uint32), want.view(np.uint32))


def test_elementwise_parity(gpu):
    n = 1 << 16
    g = synth.normal(4, "g", n, 0.0, 4.0)
    u = synth.normal(5, "u", n, 0.0, 1.0)
    dg, du = dev(g), dev(u)
    out = torch.empty_like(dg)
    E.swiglu(dg.data_ptr(), du.data_ptr(), out.data_ptr(), n, _stream())
    np.testing.assert_allclose(host(out), O.swiglu(g, u), rtol=4e-7, atol=1e-37)
    E.gelu_tanh(dg.data_ptr(), du.data_ptr(), out.data_ptr(), n, _stream())
    want = np.array([O.gelu_tanh(float(x)) for x in g[:4096]], np.float32) * u[:4096]
    # tanhf differs by an ulp between libm and the device; 1 + tanh(z) cancels for z << 0, so the
    # comparison is absolute against the unit-scale terms.
    np.testing.assert_allclose(host(out)[:4096], want, rtol=4e-6, atol=2e-7)
    E.residual_add(dg.data_ptr(), du.data_ptr(), out.data_ptr(), n, _stream())
    assert np.array_equal(host(out).view(np.uint32), O.residual_add(g, u).view(np.uint32))
    s = synth.normal(6, "s", 1000, 0.0, 3.0)
    ds = dev(s)
    so = torch.empty_like(ds)
    E.softmax(ds.data_ptr(), so.data_ptr(), s.size, _stream())
    np.testing.assert_allclose(host(so), O.softmax(s), rtol=2e-6, atol=1e-12)


def test_argmax(gpu):
    x = synth.normal(7, "lg", 32000, 0.0, 1.0)
    x[123] = x[31000] = 10.0  # tie: first index wins
    dx = dev(x)
    assert E.argmax(dx.data_ptr(), x.size, _stream()) == O.argmax(x) == 123
    x[5] = np.nan
    with pytest.raises(E.EngineError) as e:
        E.argmax(dev(x).data_ptr(), x.size, _stream())
    assert e.value.kind == "Sampling"
    with pytest.raises(E.EngineError):
        E.argmax(dx.data_ptr(), 0, _stream())


@pytest.mark.parametrize("dt,k,n", [(E.Q4K, 4096, 256), (E.Q6K, 4096, 256)])
def test_matvec_nan_input_propagates(gpu, dt, k, n):
    """The reference's f32 dot carries a NaN activation into every output it touches (src/ops/
    matmul.rs:176-204: acc += a * w, and NaN != 0 so the zero-skip does not drop it); the decode
    matvec must do the same, so a NaN reaches the logits and the greedy step reports it."""
    w = _weights(dt, k, n, 3)
    a = synth.normal(4, f"a{k}", k, 0.0, 1.0).reshape(1, k)
    a[0, 77] = np.nan
    dw, da = dev(w.view(np.uint8)), dev(a)
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    E.matmul(da.data_ptr(), 1, k, dt, dw.data_ptr(), dw.numel(), n, out.data_ptr(), _stream())
    assert np.all(np.isnan(host(out)))
