"""The no-allocation decode attention entry point (iek_dev_attention_decode_noalloc) against the
allocating one (iek_dev_attention_decode), through the C ABI: identical kernels and launch shapes,
so the outputs must be bit-identical. Two calls in a row, the second with a smaller input (fewer
heads, a shorter cache), show that the shared per-device scratch carries nothing over from the
previous call; a shape whose partials exceed the scratch is rejected with IEK_ERR_OP. Captured
in a HIP graph after a warm-up call (which resolves the scratch address), the entry point replays
bit-identically, with other work on the device between the replays.
"""
import math

import numpy as np
import pytest

from inference_engine_rust_amd import engine as E

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _case(n_heads, n_kv, hd, max_len, total, kv_f32, seed):
    rng = np.random.default_rng(seed)
    dt = torch.float32 if kv_f32 else torch.float16
    q = torch.from_numpy(rng.standard_normal(n_heads * hd).astype(np.float32)).to("cuda")
    kc = torch.from_numpy(rng.standard_normal((n_kv, max_len, hd)).astype(np.float32)).to("cuda", dt)
    vc = torch.from_numpy(rng.standard_normal((n_kv, max_len, hd)).astype(np.float32)).to("cuda", dt)
    return q, kc, vc


@pytest.mark.parametrize("kv_f32", [False, True])
def test_noalloc_matches_allocating_entry_point(gpu, kv_f32):
    stream = torch.cuda.current_stream().cuda_stream
    kvdt = E.F32 if kv_f32 else E.F16
    # second call smaller: fewer heads, shorter cache, fewer live keys, and a window
    for n_heads, n_kv, hd, max_len, total, window, seed in [(32, 8, 128, 4096, 3000, 0, 1),
                                                            (8, 1, 256, 700, 520, 256, 2)]:
        q, kc, vc = _case(n_heads, n_kv, hd, max_len, total, kv_f32, seed)
        scale = 1.0 / math.sqrt(hd)
        want = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
        got = torch.full((n_heads * hd,), float("nan"), dtype=torch.float32, device="cuda")
        E.attention_decode(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kvdt, n_heads, n_kv, hd, max_len, total,
                           window, scale, want.data_ptr(), stream)
        E.attention_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kvdt, n_heads, n_kv, hd, max_len,
                                   total, window, scale, got.data_ptr(), stream)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (n_heads, hd, float((got - want).abs().max()))


def test_noalloc_rejects_oversize(gpu):
    q, kc, vc = _case(8, 1, 64, 128, 100, True, 3)
    out = torch.empty(8 * 64, dtype=torch.float32, device="cuda")
    # 64 heads x 512 slices x 514 floats = 64 MiB of partials > the 16 MiB scratch (checked on the
    # host before any launch, so the small buffers above are never indexed by it)
    with pytest.raises(E.EngineError) as e:
        E.attention_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), E.F32, 64, 8, 512, 32768, 10, 0, 1.0,
                                   out.data_ptr())
    assert e.value.kind == "Op" and "scratch" in str(e.value)


def test_noalloc_replays_from_a_captured_graph(gpu):
    n_heads, n_kv, hd, max_len, total, window = 32, 8, 128, 2048, 1500, 0
    q, kc, vc = _case(n_heads, n_kv, hd, max_len, total, True, 4)
    scale = 1.0 / math.sqrt(hd)
    want = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
    got = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
    E.attention_decode(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), E.F32, n_heads, n_kv, hd, max_len, total, window,
                       scale, want.data_ptr(), torch.cuda.current_stream().cuda_stream)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up: resolves the scratch address before the capture
        E.attention_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), E.F32, n_heads, n_kv, hd, max_len,
                                   total, window, scale, got.data_ptr(), side.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side, capture_error_mode="thread_local"):
        E.attention_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), E.F32, n_heads, n_kv, hd, max_len,
                                   total, window, scale, got.data_ptr(), side.cuda_stream)
    for i in range(4):
        got.fill_(float("nan"))
        # other work on the device between replays, including the allocating entry point
        other = torch.empty_like(want)
        E.attention_decode(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), E.F32, n_heads, n_kv, hd, max_len, total // 2,
                           window, scale, other.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (i, float((got - want).abs().max()))
