"""Kernel parity on the GPU: the bf16 matvec at the model's real shapes and GQA decode attention,
against the CPU oracle (cpu_inference.rs:225-257 matvec/dot_bf16, :144-162 attention)."""
import numpy as np
import pytest

import oracle
import qe

pytestmark = pytest.mark.gpu

# (rows, cols) = (out, in): q, k/v, o, gate/up, down, lm_head, fused q|k|v, fused gate|up
SHAPES = [(2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072), (151936, 1024),
          (4096, 1024), (6144, 1024), (7, 8), (65, 520), (33, 4104),
          # one GPU's share under 8-way tensor parallelism (q, k/v, o, gate|up, down, lm_head)
          (256, 1024), (128, 1024), (1024, 256), (768, 1024), (1024, 384), (18992, 1024)]


def bf16_rne(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f64(w: np.ndarray) -> np.ndarray:
    return (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def run_matvec(w, x):
    import torch
    wt = torch.from_numpy(w.view(np.int16)).cuda()
    xt = torch.from_numpy(x).cuda()
    out = torch.full((w.shape[0],), float("nan"), device="cuda")
    qe.op_matvec_bf16(wt, xt, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_matches_oracle(gpu, rows, cols):
    rng = np.random.default_rng(rows * 131 + cols)
    w = bf16_rne(rng.normal(0, 0.02, size=(rows, cols)))
    x = rng.standard_normal(cols).astype(np.float32)
    got = run_matvec(w, x)
    ref32 = oracle.matvec(w, x)
    wf = bf16_to_f64(w)
    ref64 = wf @ x.astype(np.float64)
    mag = np.abs(wf) @ np.abs(x.astype(np.float64))
    # f32 accumulation error bound, loose in n but tight against any indexing mistake
    bound = 4e-7 * np.sqrt(cols) * mag + 1e-7
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - ref64) <= bound), float(np.max(np.abs(got - ref64) / bound))
    assert np.max(np.abs(got - ref32)) < 1e-4


@pytest.mark.parametrize("rows,cols", [(2048, 1024), (1024, 3072), (151936, 1024), (9, 16)])
def test_matvec_exact_on_small_integers(gpu, rows, cols):
    # small-integer weights and inputs make every product and partial sum exact in f32, so any
    # order of accumulation gives the oracle's value bit for bit
    rng = np.random.default_rng(rows + cols)
    wi = rng.integers(-3, 4, size=(rows, cols)).astype(np.float32)
    x = rng.integers(-4, 5, size=cols).astype(np.float32)
    w = bf16_rne(wi)
    got = run_matvec(w, x)
    ref = oracle.matvec(w, x)
    np.testing.assert_array_equal(got, ref)


def run_attention(q, k_pm, v_pm, n_heads, n_kv, n_splits, stride_pad=3):
    """k_pm, v_pm position-major [n_pos][n_kv*128] (the oracle's layout)."""
    import torch
    n_pos = k_pm.shape[0]
    D = 128
    stride = n_pos + stride_pad
    k_dev = np.zeros((n_kv, stride, D), np.float32)
    v_dev = np.zeros((n_kv, stride, D), np.float32)
    k_dev[:, :n_pos] = k_pm.reshape(n_pos, n_kv, D).transpose(1, 0, 2)
    v_dev[:, :n_pos] = v_pm.reshape(n_pos, n_kv, D).transpose(1, 0, 2)
    kt, vt, qt = (torch.from_numpy(a).cuda() for a in (k_dev, v_dev, q))
    out = torch.full((n_heads * D,), float("nan"), device="cuda")
    work = torch.zeros(qe.op_attention_work_bytes(n_heads, n_kv, n_pos), dtype=torch.uint8, device="cuda")
    qe.op_attention(qt, kt, vt, out, n_pos, n_heads, n_kv, work, n_splits=n_splits)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("n_pos", [1, 2, 5, 16, 17, 64, 128, 129, 258, 500, 512, 2048, 8192, 32768])
@pytest.mark.parametrize("n_splits", [0, 1, 7, 128])
def test_attention_matches_oracle(gpu, n_pos, n_splits):
    # runs of 1..n_pos positions: one 64-position tile or many per workgroup, runs past the last
    # position (n_splits > n_pos) write empty partials that the merge must weigh 0; n_splits = 1
    # at 32768 is the single pass of config 3 (one workgroup per KV head over all positions)
    rng = np.random.default_rng(n_pos)
    n_kv, G, D = 8, 2, 128
    n_heads = n_kv * G
    q = rng.standard_normal(n_heads * D).astype(np.float32)
    k = rng.standard_normal((n_pos, n_kv * D)).astype(np.float32)
    v = rng.standard_normal((n_pos, n_kv * D)).astype(np.float32)
    ref = oracle.attention(q, k, v, n_heads, n_kv, D)
    got = run_attention(q, k, v, n_heads, n_kv, n_splits)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, ref, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("G", [1, 4, 8])
def test_attention_group_sizes(gpu, G):
    rng = np.random.default_rng(100 + G)
    n_kv, D, n_pos = 2, 128, 77
    n_heads = n_kv * G
    q = rng.standard_normal(n_heads * D).astype(np.float32)
    k = rng.standard_normal((n_pos, n_kv * D)).astype(np.float32)
    v = rng.standard_normal((n_pos, n_kv * D)).astype(np.float32)
    ref = oracle.attention(q, k, v, n_heads, n_kv, D)
    for splits in (0, 1, 3):
        got = run_attention(q, k, v, n_heads, n_kv, splits)
        np.testing.assert_allclose(got, ref, atol=2e-5, rtol=1e-4)


def test_attention_single_position_is_v(gpu):
    # one position: softmax weight 1, output = v (cpu_inference.rs:157-161)
    rng = np.random.default_rng(5)
    q = rng.standard_normal(16 * 128).astype(np.float32)
    k = rng.standard_normal((1, 8 * 128)).astype(np.float32)
    v = rng.standard_normal((1, 8 * 128)).astype(np.float32)
    got = run_attention(q, k, v, 16, 8, 0).reshape(16, 128)
    vv = v.reshape(8, 128)
    np.testing.assert_allclose(got, vv[np.arange(16) // 2], atol=1e-6, rtol=1e-6)


def test_read_sum(gpu):
    import torch
    n = 1 << 24
    src = torch.ones(n, device="cuda")
    part = torch.zeros(2048, device="cuda")
    qe.op_read_sum(src, part, 2048)
    torch.cuda.synchronize()
    assert float(part.double().sum()) == float(n)


@pytest.mark.parametrize("n,grid", [(1 << 24, 2048), ((1 << 20) + 12, 777), (4, 3)])
def test_read_sum_nt(gpu, n, grid):
    # every float read exactly once over ranges that do not split evenly (workgroups with 0 or 1
    # float4s included); the values keep each partial sum exact in f32
    import torch
    src = (torch.arange(n, device="cuda") % 7).float()
    part = torch.full((grid,), float("nan"), device="cuda")
    qe.op_read_sum_nt(src, part, grid)
    torch.cuda.synchronize()
    assert float(part.double().sum()) == float(src.double().sum())
