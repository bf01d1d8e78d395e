"""rusty_hip_attention_noalloc (device buffers, fixed device scratch, no
allocation) against rusty_hip_attention on the same inputs, in both attention
orders, on two calls in a row with the second smaller, and its size limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["exact", "fast"])
def mode(request, hip):
    prev = hip.attention_mode(request.param)
    yield request.param
    hip.attention_mode(prev)


CASES = [  # (heads, n_kv, head_dim, slots, start, end, sinks)
    (32, 8, 128, 4100, 0, 4095, False),
    (8, 2, 64, 128, 0, 300, True),  # a 128-slot ring walked from slot 0 (gpt-oss full layer)
    (40, 8, 128, 700, 3, 611, False),
]


def _inputs(heads, n_kv, hd, slots, seed, sinks):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(heads * hd).astype(np.float32)
    k = rng.standard_normal(slots * n_kv * hd).astype(np.float32)
    v = rng.standard_normal(slots * n_kv * hd).astype(np.float32)
    s = (rng.standard_normal(heads) * 2).astype(np.float32) if sinks else None
    return q, k, v, s


def test_noalloc_equals_attention_two_calls(hip, mode):
    import torch
    dev = torch.device("cuda:0")
    for i, (heads, n_kv, hd, slots, st, en, sk) in enumerate(CASES):
        q, k, v, s = _inputs(heads, n_kv, hd, slots, 100 + i, sk)
        kv_mul = heads // n_kv
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        ref = np.zeros(heads * hd, np.float32)
        if sk:
            assert hip.attention_with_sink_into(q, k, v, s, ref, heads, kv_mul, hd, hd, n_kv * hd, n_kv * hd, slots,
                                                st, en, scale)
        else:
            assert hip.attention_into(q, k, v, ref, heads, kv_mul, hd, hd, n_kv * hd, n_kv * hd, slots, st, en, scale)
        tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
        ts = torch.from_numpy(s).to(dev) if sk else None
        out = torch.full((heads * hd,), float("nan"), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        assert hip.attention_noalloc_dev(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), ts.data_ptr() if sk else 0,
                                         out.data_ptr(), heads, kv_mul, hd, hd, n_kv * hd, n_kv * hd, slots, st, en,
                                         scale)
        got = out.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (i, mode, np.max(np.abs(got - ref)))


def test_noalloc_rejects_oversize_and_bad_args(hip):
    import torch
    dev = torch.device("cuda:0")
    heads, n_kv, hd, slots = 64, 8, 64, 32768
    tq = torch.zeros(heads * hd, device=dev)
    tk = torch.zeros(slots * n_kv * hd, device=dev)
    out = torch.zeros(heads * hd, device=dev)
    torch.cuda.synchronize()
    # 64 heads over 32768 positions needs ~25 MB of exact-order scratch: refused
    prev = hip.attention_mode("exact")
    try:
        assert not hip.attention_noalloc_dev(tq.data_ptr(), tk.data_ptr(), tk.data_ptr(), 0, out.data_ptr(), heads,
                                             8, hd, hd, n_kv * hd, n_kv * hd, slots, 0, slots - 1, 0.125)
        # the same call over 8192 positions fits
        assert hip.attention_noalloc_dev(tq.data_ptr(), tk.data_ptr(), tk.data_ptr(), 0, out.data_ptr(), heads,
                                         8, hd, hd, n_kv * hd, n_kv * hd, slots, 0, 8191, 0.125)
    finally:
        hip.attention_mode(prev)
    lib = hip.lib
    assert lib.rusty_hip_attention_noalloc(None, 4, tk.data_ptr(), 4, tk.data_ptr(), 4, None, 0, out.data_ptr(), 4,
                                           1, 1, 64, 64, 64, 64, 1, 0, 0, 0.125, 0) == 0


def test_noalloc_allocates_no_device_memory(hip, mode):
    """The property the entry point exists for: after one warm-up call, calls
    of every case leave the device's free memory exactly where it was."""
    import torch
    dev = torch.device("cuda:0")
    bufs = []
    for i, (heads, n_kv, hd, slots, st, en, sk) in enumerate(CASES):
        q, k, v, s = _inputs(heads, n_kv, hd, slots, 200 + i, sk)
        t = [torch.from_numpy(a).to(dev) for a in (q, k, v)]
        t.append(torch.from_numpy(s).to(dev) if sk else None)
        t.append(torch.zeros(heads * hd, dtype=torch.float32, device=dev))
        bufs.append(t)
    torch.cuda.synchronize()

    def run_all():
        for (heads, n_kv, hd, slots, st, en, sk), (tq, tk, tv, ts, out) in zip(CASES, bufs):
            scale = np.float32(1.0) / np.sqrt(np.float32(hd))
            assert hip.attention_noalloc_dev(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                                             ts.data_ptr() if sk else 0, out.data_ptr(), heads, heads // n_kv, hd,
                                             hd, n_kv * hd, n_kv * hd, slots, st, en, scale)

    run_all()  # warm-up: library initialisation and kernel loading happen here
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        run_all()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)
