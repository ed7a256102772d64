"""The drop-in modules reject bad inputs with the reference's messages
(RuntimeError, message naming the entry point) before any device work."""
import pytest
import torch

from bc_mamba_amd import extract_events_cuda as ee
from bc_mamba_amd import restore_dense_cuda_nodecay as rd
from bc_mamba_amd import selective_scan_cuda as ssc
from bc_mamba_amd import selective_scan_interface as ssi

i32 = torch.int32


@pytest.fixture
def fake_cuda(monkeypatch):
    """Lets host tensors pass the device check so the later checks are
    reached; every case below fails before any device work."""
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: True))


def _scan_inputs(E=5, NC=2, dim=2, N=4):
    return dict(u_flat=torch.randn(E), k_flat=torch.ones(E, dtype=i32), cu_seqlens=torch.tensor([0, 2, 5], dtype=i32),
                max_seqlen=3, dt_idle=torch.rand(dim), dt_active=torch.rand(dim), A=-torch.rand(dim, N),
                B=torch.randn(dim, N), C=torch.randn(dim, N))


def test_scan_rejects_host_tensors():
    with pytest.raises(RuntimeError, match="selective_scan_fwd_flat_ch: all tensors must be CUDA tensors"):
        ssc.fwd_flat_ch(**_scan_inputs(), is_depthwise_bc=True)


@pytest.mark.parametrize("field,bad,msg", [
    ("k_flat", torch.ones(5, dtype=torch.int64), "k_flat must be int32"),
    ("A", -torch.rand(2, 4, dtype=torch.float64), "A must be float32"),
    ("u_flat", torch.randn(5, dtype=torch.float64), "u_flat must be fp16/bf16/fp32"),
    ("A", -torch.rand(2, 300), "dstate must be <= 256"),
])
def test_scan_dtype_and_shape_checks(field, bad, msg, fake_cuda):
    args = _scan_inputs()
    args[field] = bad
    with pytest.raises(RuntimeError, match=msg):
        ssc.fwd_flat_ch(**args, is_depthwise_bc=True)


def test_scan_mode_shape_checks(fake_cuda):
    """Legacy, tiled and pointwise modes check their operand shapes like
    selective_scan.cpp:760-776, 840-848, 969-990 before any device work."""
    a = _scan_inputs()
    with pytest.raises(RuntimeError, match="B must have shape \\(4, 5\\)"):
        ssc.fwd_flat_ch(**a, is_depthwise_bc=False)  # [dim, dstate] is not a legacy [dstate, E] operand
    leg = dict(a, B=torch.randn(4, 5)[:, :5], C=torch.randn(5, 4).t())
    with pytest.raises(RuntimeError, match="stride\\(1\\) == 1"):
        ssc.fwd_flat_ch(**leg, is_depthwise_bc=False)
    with pytest.raises(RuntimeError, match="tiled B/C must be 3-D"):
        ssc.fwd_flat_ch(**a, tile_offsets=torch.zeros(2, dtype=i32), tile_chunk_size=4)
    til = dict(a, B=torch.randn(3, 4, 8), C=torch.randn(3, 4, 8))
    with pytest.raises(RuntimeError, match="dim-2 must equal tile_chunk_size"):
        ssc.fwd_flat_ch(**til, tile_offsets=torch.zeros(2, dtype=i32), tile_chunk_size=4)
    with pytest.raises(RuntimeError, match="pw_B must be \\[dim, dim\\]"):
        ssc.fwd_flat_ch(**a, is_depthwise_bc=True, pw_B=torch.eye(3), pw_C=torch.eye(2))
    with pytest.raises(RuntimeError, match="must have shape \\(4, 5\\) or \\(4, 2\\)"):
        ssc.bwd_flat_ch(**dict(a, B=torch.randn(4, 3), C=torch.randn(4, 5)), dout_flat=torch.randn(5),
                        x=torch.zeros(2, 1, 8), is_depthwise_bc=False)


def test_bwd_checks_x_chunks():
    args = _scan_inputs()
    with pytest.raises(RuntimeError, match="selective_scan_bwd_flat_ch"):
        ssc.bwd_flat_ch(**args, dout_flat=torch.randn(5, dtype=torch.float16), x=torch.zeros(2, 1, 8),
                        is_depthwise_bc=True)


def test_restore_checks():
    y, t, cu = torch.randn(4), torch.tensor([0, 3, 1, 2], dtype=i32), torch.tensor([0, 2, 4], dtype=i32)
    with pytest.raises(RuntimeError, match="restore_dense_fwd: all tensors must be on CUDA"):
        rd.restore_dense_fwd(y, t, cu, 1, 8)
    with pytest.raises(RuntimeError, match="restore_dense_fwd: time_steps must be int32"):
        rd.restore_dense_fwd(y, t.long(), cu, 1, 8)
    with pytest.raises(RuntimeError, match="restore_dense_fwd: y_flat must be fp32, fp16, or bf16"):
        rd.restore_dense_fwd(y.double(), t, cu, 1, 8)
    with pytest.raises(RuntimeError, match="restore_dense_bwd: all tensors must be on CUDA"):
        rd.restore_dense_bwd(torch.zeros(2, 8), t, cu, 1, 8)


def test_restore_shape_checks(fake_cuda):
    t, cu = torch.tensor([0, 3, 1, 2], dtype=i32), torch.tensor([0, 2, 4], dtype=i32)
    with pytest.raises(RuntimeError, match="restore_dense_bwd: dout must be 3-D"):
        rd.restore_dense_bwd(torch.zeros(2, 8), t, cu, 1, 8)
    with pytest.raises(RuntimeError, match="restore_dense_fwd: n_channels \\(B\\*D\\) must be divisible by dim"):
        rd.restore_dense_fwd(torch.zeros(4), t, cu, 3, 8)
    with pytest.raises(RuntimeError, match="bf16 input only supports bf16 output"):
        rd.restore_dense_fwd(torch.zeros(4, dtype=torch.bfloat16), t, cu, 1, 8, torch.float32)


def test_restore_proj_checks():
    """The restore -> out_proj op is fp32 with the nn.Linear weight layout;
    other inputs are refused before any device work."""
    idx = (torch.zeros(2, 32, dtype=i32), torch.zeros(2, 2, dtype=i32), 1)
    y, w = torch.randn(4), torch.randn(3, 2)
    with pytest.raises(RuntimeError, match="restore_proj_fwd_indexed: fp32 y_flat and weight"):
        rd.restore_proj_fwd_indexed(y.bfloat16(), idx, 2, 2, 8, w)
    with pytest.raises(RuntimeError, match="restore_proj_fwd_indexed: fp32 bias"):
        rd.restore_proj_fwd_indexed(y, idx, 2, 2, 8, w, torch.zeros(3, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="restore_proj_fwd_indexed: weight \\[d_model, dim\\]"):
        rd.restore_proj_fwd_indexed(y, idx, 2, 2, 8, torch.randn(3, 5))


def test_extract_checks():
    with pytest.raises(RuntimeError, match="base_input must be CUDA"):
        ee.extract_base_events(torch.zeros(1, 2, 3), 0.5)
    with pytest.raises(RuntimeError, match="mask must be a CUDA tensor"):
        ee.extract_events(torch.zeros(1, 2, 3, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="gather_events_fwd: x must be a CUDA tensor"):
        ee.gather_events_fwd(torch.zeros(1, 2, 3), torch.zeros(1, dtype=i32), torch.zeros(1, dtype=i32))
    with pytest.raises(RuntimeError, match="gather_events_bwd: grad tensor must be CUDA"):
        ee.gather_events_bwd(torch.zeros(1), torch.zeros(1, dtype=i32), torch.zeros(1, dtype=i32), 1, 3)


def test_interface_exports_reference_names():
    assert callable(ssi.selective_scan_flat_ch_fn)
    assert issubclass(ssi.SelectiveScanFlatChFn, torch.autograd.Function)
    with pytest.raises(RuntimeError, match="not part of"):
        ssi.selective_scan_depthwise_bc_fn()


def test_spike_bits_and_bits_extraction_checks(fake_cuda):
    with pytest.raises(RuntimeError, match="p must be a contiguous 3-D CUDA tensor"):
        ee.spike_bits(torch.rand(4, 8), 0.5)
    with pytest.raises(RuntimeError, match="p must be fp32, fp16 or bf16"):
        ee.spike_bits(torch.rand(2, 4, 8, dtype=torch.float64), 0.5)
    bad = torch.zeros((3, 32), dtype=i32)  # rows of 2 x 2 channels need 4
    with pytest.raises(RuntimeError, match="bits must be"):
        ee.extract_events_indexed(None, 0.5, 1, None, bits=(bad, (2, 2, 64)))
    ok = torch.zeros((4, 32), dtype=i32)
    with pytest.raises(RuntimeError, match="bits need the fused fill"):
        ee.extract_events_indexed(None, 0.5, 1, None, exact_alloc=True, bits=(ok, (2, 2, 64)))


def test_conv_at_events_checks(fake_cuda):
    mem = torch.zeros(2, 2, 64)
    x = torch.zeros(2, 4, 64)[:, :, :63]  # 63 steps where the membrane has 64
    w = torch.zeros(4, 4)
    with pytest.raises(RuntimeError, match="x must be a CUDA tensor"):
        ee.extract_events_indexed(mem, 0.5, 2, x, conv=(w, None, True))
    x = torch.zeros(2, 4, 64)
    with pytest.raises(RuntimeError, match="conv needs the fused fill"):
        ee.extract_events_indexed(mem, 0.5, 2, x, exact_alloc=True, conv=(w, None, True))


def test_spike_sampler_uses_torch_off_the_gpu():
    """The fused STE head runs only on CUDA tensors; elsewhere the sampler
    computes the reference expression (same values, same gradient)."""
    from bc_mamba_amd.e_model import SpikeSamplerSurrogate
    p = torch.rand(2, 5, 3, requires_grad=True)
    s = SpikeSamplerSurrogate(mode="ste", threshold=0.4)(p)
    assert torch.equal(s, (p >= 0.4).float() + p - p) and not hasattr(s, "_bcm_event_bits")
    s.sum().backward()
    assert torch.equal(p.grad, torch.ones_like(p))


def test_split_k_projections_match_torch():
    """The projections' split-K weight gradients (8 token chunks, ordered sum)
    agree with torch's products within fp32 rounding; forward values and
    input gradients are the same products."""
    from bc_mamba_amd import projections as pj
    torch.manual_seed(0)
    M = pj.MIN_TOKENS
    x = torch.randn(2, M // 2, 48, requires_grad=True)
    w = torch.randn(40, 48, requires_grad=True)
    b = torch.randn(40, requires_grad=True)
    gy = torch.randn(2, M // 2, 40)
    y = pj.linear(x, w, b)
    y.backward(gy)
    x2, w2, b2 = (t.detach().clone().requires_grad_(True) for t in (x, w, b))
    y2 = torch.nn.functional.linear(x2, w2, b2)
    y2.backward(gy)
    assert torch.equal(y, y2) and torch.allclose(x.grad, x2.grad, rtol=1e-5, atol=1e-5)
    assert torch.allclose(w.grad, w2.grad, rtol=1e-4, atol=1e-4 * w2.grad.abs().max().item())
    assert torch.allclose(b.grad, b2.grad, rtol=1e-4, atol=1e-4 * b2.grad.abs().max().item())
    h = torch.randn(M, 24, requires_grad=True)
    wi = torch.randn(32, 24, requires_grad=True)
    g = torch.randn(32, M)
    pj.proj_tokens_last(wi, h).backward(g)
    h2, wi2 = h.detach().clone().requires_grad_(True), wi.detach().clone().requires_grad_(True)
    (wi2 @ h2.t()).backward(g)
    assert torch.allclose(wi.grad, wi2.grad, rtol=1e-4, atol=1e-4 * wi2.grad.abs().max().item())
    assert torch.allclose(h.grad, h2.grad, rtol=1e-5, atol=1e-5)
