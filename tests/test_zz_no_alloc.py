"""qe_op_attention_static, the allocation-free variant of qe_op_attention: through the C ABI, its
output equals qe_op_attention's (same kernels, partials in the library's static device array
instead of a caller work buffer) bit for bit, on two calls in a row, the second smaller, and a
call beyond the array's size is refused before any launch."""
import ctypes

import numpy as np
import pytest

import qe

pytestmark = pytest.mark.gpu


def static_fn():
    f = qe.lib().qe_op_attention_static
    vp, u64 = ctypes.c_void_p, ctypes.c_uint64
    f.restype = ctypes.c_int
    f.argtypes = [vp, vp, vp, vp, u64, u64, u64, u64, ctypes.c_uint32, vp]
    return f


def run_pair(torch, n_pos, kv_stride, n_heads, n_kv, n_splits, seed):
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal(n_heads * 128).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.standard_normal((n_kv, kv_stride, 128)).astype(np.float32)).cuda()
    v = torch.from_numpy(rng.standard_normal((n_kv, kv_stride, 128)).astype(np.float32)).cuda()
    ref = torch.full((n_heads * 128,), float("nan"), device="cuda")
    got = torch.full((n_heads * 128,), float("nan"), device="cuda")
    work = torch.empty(qe.op_attention_work_bytes(n_heads, n_kv, n_pos) // 4 + 64, device="cuda")
    qe.op_attention(q, k, v, ref, n_pos, n_heads, n_kv, work, n_splits=n_splits)
    rc = static_fn()(q.data_ptr(), k.data_ptr(), v.data_ptr(), got.data_ptr(), n_pos, kv_stride, n_heads, n_kv,
                     n_splits, None)
    assert rc == qe.QE_OK, qe.lib().qe_last_error()
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


def test_static_attention_matches_work_buffer_variant(gpu):
    import torch
    # a large call (128 runs of 64 positions x 16 heads: every row of the static area), then a
    # smaller one that reuses the same rows with fewer runs and positions
    for n_pos, stride, nh, nkv, sp, seed in [(8192, 8200, 16, 8, 0, 1), (300, 512, 16, 8, 0, 2),
                                            (77, 77, 8, 8, 3, 3)]:
        ref, got = run_pair(torch, n_pos, stride, nh, nkv, sp, seed)
        assert np.all(np.isfinite(got))
        np.testing.assert_array_equal(got, ref)


def test_static_attention_under_graph_capture(gpu):
    """after one eager call on the device (it looks up the array's address), the op is captured in a
    graph; each replay, with new q values written eagerly in between, equals qe_op_attention's
    output on the same inputs bit for bit"""
    import torch
    n_pos, stride, nh, nkv = 700, 704, 16, 8
    rng = np.random.default_rng(11)
    qs = torch.from_numpy(rng.standard_normal((4, nh * 128)).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.standard_normal((nkv, stride, 128)).astype(np.float32)).cuda()
    v = torch.from_numpy(rng.standard_normal((nkv, stride, 128)).astype(np.float32)).cuda()
    q = qs[0].clone()
    got = torch.full((nh * 128,), float("nan"), device="cuda")
    ref = torch.empty_like(got)
    work = torch.empty(qe.op_attention_work_bytes(nh, nkv, n_pos) // 4 + 64, device="cuda")
    f = static_fn()

    def call():
        rc = f(q.data_ptr(), k.data_ptr(), v.data_ptr(), got.data_ptr(), n_pos, stride, nh, nkv, 0,
               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == qe.QE_OK, qe.lib().qe_last_error()

    call()  # the eager first call on this device
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for i in range(4):
        q.copy_(qs[i])
        got.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        qe.op_attention(q, k, v, ref, n_pos, nh, nkv, work)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy(), err_msg=f"replay {i}")


def test_static_attention_refuses_oversized_calls(gpu):
    import torch
    q = torch.zeros(32 * 128, device="cuda")
    kv = torch.zeros((8, 8192, 128), device="cuda")
    out = torch.zeros(32 * 128, device="cuda")
    # 32 q heads x 128 runs = 4096 partial rows > 2048
    rc = static_fn()(q.data_ptr(), kv.data_ptr(), kv.data_ptr(), out.data_ptr(), 8192, 8192, 32, 8, 0, None)
    assert rc == qe.QE_ERR_ARG and b"static work area" in qe.lib().qe_last_error()
