"""Per-kernel parity of libquail_hip.so against the CPU oracle (MI355X only).

Inputs are seeded and built on the CPU; each kernel runs through the C ABI
(quail_amd.kernels -> quail_amd._hip) and is compared with oracle.ops on the
same inputs. Bars: integer/index work bit-exact; fp8 quantization bit-exact
where the inputs of the rounding are computed identically (group quant),
otherwise at most 1 e4m3 step on a tiny fraction of elements (sums taken in
a different order move values across a rounding midpoint); attention
max-abs <= 2e-3 against fp32.
"""

import math

import pytest
import torch

from oracle import ops as ref
from quail_amd import kernels as K
from quail_amd import layout

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _e4m3_steps(a, b):
    """Per-element distance in e4m3 codes (monotone integer mapping)."""
    def key(q):
        u = q.view(torch.uint8).to(torch.int32)
        mag = u & 0x7F
        return torch.where(u >= 0x80, -mag, mag)
    return (key(a) - key(b)).abs()


def _check_quant(q_gpu, s_gpu, q_ref, s_ref, *, max_frac_off=2e-4, scale_rtol=1e-6):
    q_gpu, s_gpu = q_gpu.cpu(), s_gpu.cpu()
    assert torch.allclose(s_gpu, s_ref, rtol=scale_rtol, atol=0), \
        f"scales differ: max rel {((s_gpu - s_ref).abs() / s_ref).max().item()}"
    steps = _e4m3_steps(q_gpu, q_ref)
    assert steps.max().item() <= 1, f"fp8 codes differ by {steps.max().item()} steps"
    frac = (steps > 0).float().mean().item()
    assert frac <= max_frac_off, f"{frac:.2e} of fp8 codes differ"


@pytest.mark.parametrize("H", [1024, 2560, 5120, 8192])
def test_add_rmsnorm_quant_fused_and_plain(H):
    g = _gen(1)
    T = 37
    x = (torch.randn(T, H, generator=g) * 2).to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    eps = 1e-6
    q_ref, s_ref, r_ref = ref.add_rms_norm_quant(x, r, w, eps)
    r_gpu = r.to(DEV)
    q, s = K.add_rmsnorm_quant(x.to(DEV), w.to(DEV), eps, residual=r_gpu)
    assert torch.equal(r_gpu.cpu(), r_ref), "residual write-back must be bit-exact"
    _check_quant(q, s, q_ref, s_ref)
    # layer-0 path: vLLM rms_norm (bf16 out) then group quant
    q_ref, s_ref = ref.norm_quant_plain(x, w, eps)
    q, s = K.add_rmsnorm_quant(x.to(DEV), w.to(DEV), eps)
    _check_quant(q, s, q_ref, s_ref, max_frac_off=2e-3)


@pytest.mark.parametrize("ue8m0", [False, True])
def test_group_quant_bit_exact(ue8m0):
    g = _gen(2)
    x = (torch.randn(53, 4096, generator=g) * 3).to(torch.bfloat16)
    x[3] = 0  # an all-zero row takes the 1e-10 floor
    q_ref, s_ref = ref.group_quant(x.float(), ue8m0)
    q, s = K.group_quant(x.to(DEV), ue8m0)
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


def test_group_quant_division_is_exact_over_wide_magnitudes():
    """y / scale is formed as y * (1 / scale) in fp64 and rounded once to fp32;
    it must equal torch's fp32 division everywhere, so 16k groups of values
    spread over 2^-30 .. 2^30, each group with its own non-power-of-two
    scale, quantize bit for bit as the oracle does."""
    g = _gen(21)
    rows = 4096
    mag = torch.pow(2.0, torch.randint(-30, 31, (rows, 1), generator=g).float())
    x = (torch.randn(rows, 512, generator=g) * mag * (1 + torch.rand(rows, 512, generator=g)))
    x = x.to(torch.bfloat16)
    q_ref, s_ref = ref.group_quant(x.float())
    q, s = K.group_quant(x.to(DEV))
    assert torch.equal(s.cpu(), s_ref)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


def test_e4m3_encoding_matches_torch_at_every_midpoint():
    # Rows whose amax is 448 quantize with scale exactly 1, so the kernel's
    # e4m3 encoder sees the raw values: every finite e4m3 value, every
    # midpoint between neighbours (4 significant bits: exact in bf16) and the
    # bf16 values either side of each midpoint, both signs. torch's CPU
    # float8_e4m3fn cast (round to nearest even) is the expected result.
    codes = torch.arange(0, 0x7F, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float()
    mids = ((vals[:-1] + vals[1:]) / 2).to(torch.bfloat16)
    assert torch.equal(mids.float(), (vals[:-1] + vals[1:]) / 2)
    bits = mids.view(torch.int16)
    up = (bits + 1).view(torch.bfloat16)
    down = (bits - 1).view(torch.bfloat16)
    pool = torch.cat([vals.to(torch.bfloat16), mids, up, down])
    pool = torch.cat([pool, -pool])
    per_row = 127
    rows = -(-pool.numel() // per_row)
    flat = torch.zeros(rows * per_row, dtype=torch.bfloat16)
    flat[:pool.numel()] = pool
    x = torch.zeros(rows, 128, dtype=torch.bfloat16)
    x[:, :per_row] = flat.view(rows, per_row)
    x[:, per_row] = 448.0
    q_ref, s_ref = ref.group_quant(x.float())
    assert torch.all(s_ref == 1.0)
    q, s = K.group_quant(x.to(DEV))
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8))


def test_fused_epilogue_encoder_saturates_just_above_448():
    """The fused epilogues' encoder has no +-448 clamp: a value no larger
    than its group's amax gives |y / scale| <= 448 (1 + 2^-24), which fp32
    rounds to at most 448 + 2^-15. Every value in (448, 464] must encode as
    +-448 (0x7e / 0xfe), never as the NaN code, and values up to 448 as
    torch's float8_e4m3fn cast does."""
    above = torch.tensor([448 + 2 ** -15, 448 + 2 ** -10, 450.0, 455.5, 463.9, 464.0],
                         dtype=torch.float32)
    assert above[0].item() > 448 and above[0].item() == 448 + 2 ** -15
    below = torch.tensor([448.0, 447.99, 440.0, 432.0, 0.0, 1.0, 2 ** -9, 2 ** -10],
                         dtype=torch.float32)
    x = torch.cat([above, -above, below, -below])
    got = K.e4m3_encode(x.to(DEV)).cpu()
    n = above.numel()
    assert got[:n].tolist() == [0x7E] * n, [hex(v) for v in got[:n].tolist()]
    assert got[n:2 * n].tolist() == [0xFE] * n, [hex(v) for v in got[n:2 * n].tolist()]
    rest = x[2 * n:]
    assert torch.equal(got[2 * n:], rest.to(torch.float8_e4m3fn).view(torch.uint8))


def test_silu_mul_quant():
    g = _gen(3)
    T, I = 29, 9728
    gu = (torch.randn(T, 2 * I, generator=g) * 2).to(torch.bfloat16)
    q_ref, s_ref = ref.silu_mul_quant(gu)
    q, s = K.silu_mul_quant(gu.to(DEV))
    _check_quant(q, s, q_ref, s_ref, max_frac_off=1e-3, scale_rtol=2e-6)


def test_qk_norm_rope():
    g = _gen(4)
    T, n_q, n_kv, d = 41, 32, 8, 128
    qkv = torch.randn(T, (n_q + 2 * n_kv) * d, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, 4000, (T,), generator=g)
    cs = ref.rope_cache(4096, d, 1e6)
    qw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    q_ref, k_ref, v_ref = ref.qk_norm_rope(qkv, pos, cs, qw, kw, 1e-6, n_q, n_kv, d)
    q, k, v = K.qk_norm_rope(qkv.to(DEV), pos.to(DEV), cs.to(DEV), qw.to(DEV),
                             kw.to(DEV), 1e-6, n_q, n_kv, d)
    assert torch.equal(v.cpu(), v_ref)
    for got, want in ((q.cpu(), q_ref), (k.cpu(), k_ref)):
        diff = (got.float() - want.float()).abs()
        ulp = want.float().abs().clamp(min=1e-30) * 2 ** -7
        assert (diff <= ulp).all(), f"max diff {diff.max().item()}"
        assert (diff > 0).float().mean() < 1e-2


@pytest.mark.parametrize("M,N,Kd", [(1, 256, 128), (300, 512, 2560), (517, 6144, 2560),
                                    (256, 2560, 9728)])
def test_fp8_gemm_nt(M, N, Kd):
    g = _gen(5)
    w = torch.randn(N, Kd, generator=g) * 0.02
    wq, ws = ref.quantize_weight_blocks(w)
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    xq, xs = ref.group_quant(x.float())
    want = ref.fp8_gemm(xq, xs, wq, ws, out_dtype=torch.float64)
    xs_dev = K.col_major_scales(M, Kd, DEV)
    xs_dev.copy_(xs)
    got = K.fp8_gemm_nt(xq.to(DEV), xs_dev, wq.to(DEV), ws.to(DEV)).cpu().double()
    err = (got - want).abs()
    tol = want.abs() * 2 ** -8 + 1e-3 * want.abs().max()
    assert (err <= tol).all(), f"max err {err.max().item()} (scale {want.abs().max().item()})"


def _gemm_inputs(seed, M, N, Kd, dev):
    """Random e4m3 activations / weights with random fp32 scales, on `dev`."""
    g = _gen(seed)
    a = (torch.randn(M, Kd, generator=g) * 2).to(torch.float8_e4m3fn).to(dev)
    w = torch.randn(N, Kd, generator=g).to(torch.float8_e4m3fn).to(dev)
    sa = K.col_major_scales(M, Kd, dev)
    sa.copy_((torch.rand(M, Kd // 128, generator=g) * 0.02 + 1e-3).to(dev))
    sw = (torch.rand(N // 128, Kd // 128, generator=g) * 0.01 + 1e-4).to(dev)
    return a, sa, w, sw


@pytest.mark.parametrize("M,N,Kd", [(4096, 4608, 1024), (2333, 19456, 384)])
def test_fp8_gemm_nt_many_tiles(M, N, Kd):
    """More tiles than compute units: each persistent workgroup walks several
    tiles, with loads running across tile boundaries. Reference: the same
    dequantized operands in an fp32 torch matmul on the GPU."""
    a, sa, w, sw = _gemm_inputs(11, M, N, Kd, DEV)
    got = K.fp8_gemm_nt(a, sa, w, sw).float()
    a32 = a.float() * sa.repeat_interleave(128, dim=1)
    w32 = w.float() * sw.repeat_interleave(128, dim=0).repeat_interleave(128, dim=1)
    want = a32 @ w32.t()
    err = (got - want).abs()
    tol = want.abs() * 2 ** -8 + 1e-3 * want.abs().max()
    assert (err <= tol).all(), f"max err {err.max().item()}"


def test_fp8_gemm_nt_is_deterministic():
    """Launches with the same inputs give the same bits: each output has one
    fixed order of MFMA products and promotions, whatever the timing of the
    DMA ring, the tile boundaries or the neighbouring workgroups (several
    tiles per workgroup, a ragged last tile row)."""
    a, sa, w, sw = _gemm_inputs(14, 8191, 9728, 1280, DEV)
    first = K.fp8_gemm_nt(a, sa, w, sw)
    for _ in range(3):
        again = K.fp8_gemm_nt(a, sa, w, sw)
        assert torch.equal(first.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("M,I,Kd", [(1, 128, 128), (300, 1024, 2560), (517, 9728, 256),
                                    (2048, 9728, 512)])
@pytest.mark.parametrize("ue8m0", [False, True])
def test_fp8_gemm_silu_quant_matches_pair(M, I, Kd, ue8m0):
    """The fused gate_up + SiLU + quant kernel equals fp8_gemm_nt followed by
    silu_mul_quant bit for bit (values and scales)."""
    a, sa, w, sw = _gemm_inputs(12 + M, M, 2 * I, Kd, DEV)
    gate_up = K.fp8_gemm_nt(a, sa, w, sw)
    q_pair, s_pair = K.silu_mul_quant(gate_up, ue8m0)
    q, s = K.fp8_gemm_silu_quant(a, sa, w, sw, ue8m0)
    assert torch.equal(s.cpu(), s_pair.cpu())
    assert torch.equal(q.view(torch.uint8).cpu(), q_pair.view(torch.uint8).cpu())


def _ue8m0_inputs(seed, M, N, Kd):
    """UE8M0-quantized weights N(0, 0.02) and activations N(0, 1) (CPU), with
    the activation scales also on the GPU in the column-major layout."""
    g = _gen(seed)
    wq, ws = ref.quantize_weight_blocks(torch.randn(N, Kd, generator=g) * 0.02, ue8m0=True)
    xq, xs = ref.group_quant(torch.randn(M, Kd, generator=g), ue8m0=True)
    mant_w, _ = torch.frexp(ws)
    mant_x, _ = torch.frexp(xs)
    assert (mant_w == 0.5).all() and (mant_x == 0.5).all()
    xs_dev = K.col_major_scales(M, Kd, DEV)
    xs_dev.copy_(xs)
    return xq, xs, xs_dev, wq, ws


@pytest.mark.parametrize("M,N,Kd", [(1, 256, 128), (300, 512, 2560), (517, 6144, 2560),
                                    (2333, 19456, 384), (256, 2560, 9728)])
def test_fp8_gemm_nt_ue8m0_matches_the_oracle(M, N, Kd):
    """UE8M0 scales applied by the MFMA's E8M0 operands: against the oracle's
    fp64 block sums (same bar as the fp32-scale kernel), and against the
    fp32-promotion kernel on the same operands, which computes the same sums
    with power-of-two (exact) promotion multipliers."""
    xq, xs, xs_dev, wq, ws = _ue8m0_inputs(30 + M, M, N, Kd)
    want = ref.fp8_gemm(xq, xs, wq, ws, out_dtype=torch.float64)
    got = K.fp8_gemm_nt(xq.to(DEV), xs_dev, wq.to(DEV), ws.to(DEV), ue8m0_scales=True)
    err = (got.cpu().double() - want).abs()
    tol = want.abs() * 2 ** -8 + 1e-3 * want.abs().max()
    assert (err <= tol).all(), f"max err {err.max().item()} (scale {want.abs().max().item()})"
    promo = K.fp8_gemm_nt(xq.to(DEV), xs_dev, wq.to(DEV), ws.to(DEV)).float()
    rel = ((got.float() - promo).norm() / promo.norm()).item()
    assert rel < 2e-3, f"relative L2 to the promotion kernel {rel}"


def test_fp8_gemm_nt_ue8m0_is_deterministic():
    xq, xs, xs_dev, wq, ws = _ue8m0_inputs(35, 4099, 6144, 1280)
    args = (xq.to(DEV), xs_dev, wq.to(DEV), ws.to(DEV))
    first = K.fp8_gemm_nt(*args, ue8m0_scales=True)
    for _ in range(3):
        again = K.fp8_gemm_nt(*args, ue8m0_scales=True)
        assert torch.equal(first.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("M,I,Kd", [(1, 128, 128), (517, 9728, 256), (2048, 9728, 512)])
def test_fp8_gemm_silu_quant_ue8m0_matches_pair(M, I, Kd):
    """The UE8M0 gate_up kernel equals its own bf16 GEMM (qh_fp8_gemm_nt_ue8m0)
    followed by silu_mul_quant(ue8m0) bit for bit."""
    xq, xs, xs_dev, wq, ws = _ue8m0_inputs(40 + M, M, 2 * I, Kd)
    args = (xq.to(DEV), xs_dev, wq.to(DEV), ws.to(DEV))
    gate_up = K.fp8_gemm_nt(*args, ue8m0_scales=True)
    q_pair, s_pair = K.silu_mul_quant(gate_up, True)
    q, s = K.fp8_gemm_silu_quant(*args, ue8m0=True, ue8m0_scales=True)
    assert torch.equal(s.cpu(), s_pair.cpu())
    assert torch.equal(q.view(torch.uint8).cpu(), q_pair.view(torch.uint8).cpu())


def test_fp8_gemm_silu_quant_oracle():
    """Against the oracle: fp64 GEMM rounded to bf16, then oracle silu_mul_quant."""
    g = _gen(13)
    M, I, Kd = 77, 256, 640
    w = torch.randn(2 * I, Kd, generator=g) * 0.05
    wq, ws = ref.quantize_weight_blocks(w)
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    xq, xs = ref.group_quant(x.float())
    gate_up = ref.fp8_gemm(xq, xs, wq, ws, out_dtype=torch.float64).to(torch.bfloat16)
    q_ref, s_ref = ref.silu_mul_quant(gate_up)
    xs_dev = K.col_major_scales(M, Kd, DEV)
    xs_dev.copy_(xs)
    q, s = K.fp8_gemm_silu_quant(xq.to(DEV), xs_dev, wq.to(DEV), ws.to(DEV))
    # the GEMM's fp32 block sums may round a bf16 input one ulp away from the
    # fp64 reference's, which moves a few outputs by one e4m3 step
    _check_quant(q, s, q_ref, s_ref, max_frac_off=2e-2, scale_rtol=1e-2)


def _paged_case(seed, n_seqs, prefix, max_suffix, n_q=32, n_kv=8, d=128):
    """Sequences sharing a `prefix`-token node, own suffixes, permuted pages."""
    g = _gen(seed)
    page = 16
    lens = torch.randint(1, max_suffix + 1, (n_seqs,), generator=g).tolist()
    prefix_pages = -(-prefix // page)
    need = prefix_pages + sum(-(-(prefix % page + L) // page) + 1 for L in lens)
    n_pages = need + 8
    perm = torch.randperm(n_pages, generator=g).tolist()
    k_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    v_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    shared = perm[:prefix_pages]
    cursor = prefix_pages
    tables, used = [], []
    for L in lens:
        total = prefix + L
        pages = list(shared[:prefix // page])
        while len(pages) * page < total:
            pages.append(perm[cursor])
            cursor += 1
        # a partially shared last prefix page is copied into the sequence's own page
        tables.append(pages)
        used.append(total)
    width = max(map(len, tables))
    table = torch.zeros(n_seqs, width, dtype=torch.int32)
    for i, p in enumerate(tables):
        table[i, :len(p)] = torch.tensor(p, dtype=torch.int32)
    cu_q = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T = int(cu_q[-1])
    q = (torch.randn(T, n_q, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    return dict(q=q, k_rows=k_rows, v_rows=v_rows, table=table,
                used=torch.tensor(used, dtype=torch.int32), cu_q=cu_q, lens=lens,
                n_kv=n_kv, max_q=max(lens))


def _run_paged(case, causal, q_rows=None):
    scale = 1 / math.sqrt(case["q"].shape[-1])
    kp = layout.k_pool_from_rows(case["k_rows"]).to(DEV)
    vp = layout.v_pool_from_rows(case["v_rows"]).to(DEV)
    n_queries = int(case["cu_q"][-1])
    out, lse = K.attention(case["q"].to(DEV), case["cu_q"].to(DEV), case["used"].to(DEV),
                           n_queries=n_queries, max_q=case["max_q"], softmax_scale=scale,
                           causal=causal, k_pool=kp, v_pool=vp, table=case["table"].to(DEV),
                           q_rows=None if q_rows is None else q_rows.to(DEV),
                           n_kv=case["n_kv"], want_lse=True)
    want, want_lse = ref.paged_attention(case["q"], case["k_rows"], case["v_rows"],
                                         case["cu_q"], case["used"], case["table"],
                                         scale, causal, q_rows=q_rows)
    return out.cpu().float(), lse.cpu(), want, want_lse


@pytest.mark.parametrize("seed,n_seqs,prefix,max_suffix", [
    (10, 8, 64, 100), (11, 5, 256, 256), (12, 3, 37, 300), (13, 16, 0, 40)])
def test_paged_attention_causal(seed, n_seqs, prefix, max_suffix):
    case = _paged_case(seed, n_seqs, prefix, max_suffix)
    got, lse, want, want_lse = _run_paged(case, causal=True)
    err = (got - want).abs().max().item()
    assert err <= 2e-3, f"max-abs {err}"
    assert torch.allclose(lse, want_lse, atol=2e-3, rtol=0)


def test_paged_attention_ignores_unread_rows():
    """Arena rows no sequence reads (past `used` in a last page, whole unused
    pages) hold NaN: the kernel must not let them into any output."""
    case = _paged_case(14, 7, 48, 90)
    page = 16
    read = torch.zeros(case["k_rows"].shape[0], dtype=torch.bool)
    for s in range(case["table"].shape[0]):
        for j in range(int(case["used"][s])):
            read[int(case["table"][s, j // page]) * page + j % page] = True
    nan_case = dict(case, k_rows=case["k_rows"].clone(), v_rows=case["v_rows"].clone())
    nan_case["k_rows"][~read] = float("nan")
    nan_case["v_rows"][~read] = float("nan")
    got, lse, want, want_lse = _run_paged(nan_case, causal=True)
    assert torch.isfinite(got).all() and torch.isfinite(lse).all()
    assert (got - want).abs().max().item() <= 2e-3
    assert torch.allclose(lse, want_lse, atol=2e-3, rtol=0)


@pytest.mark.parametrize("causal,gathered", [(True, False), (False, True)])
@pytest.mark.parametrize("ue8m0", [False, True])
def test_attention_fp8_matches_quantized_bf16(causal, gathered, ue8m0):
    """The fp8-output attention equals attention (bf16) then group_quant,
    bit for bit."""
    case = _paged_case(40 + int(causal), 9, 80, 120)
    T = int(case["cu_q"][-1])
    q3, rows = case["q"], None
    if gathered:
        g = _gen(41)
        big = torch.randn(T + 30, 32, 128, generator=g).to(torch.bfloat16)
        rows = torch.randperm(T + 30, generator=g)[:T].sort().values
        big[rows] = case["q"]
        q3, rows = big, rows.to(DEV)
    kp = layout.k_pool_from_rows(case["k_rows"]).to(DEV)
    vp = layout.v_pool_from_rows(case["v_rows"]).to(DEV)
    args = dict(n_queries=T, max_q=case["max_q"], softmax_scale=1 / math.sqrt(128),
                causal=causal, k_pool=kp, v_pool=vp, table=case["table"].to(DEV),
                q_rows=rows, n_kv=case["n_kv"])
    out, _ = K.attention(q3.to(DEV), case["cu_q"].to(DEV), case["used"].to(DEV), **args)
    q_ref, s_ref = K.group_quant(out.view(T, -1), ue8m0)
    q, s = K.attention_fp8(q3.to(DEV), case["cu_q"].to(DEV), case["used"].to(DEV),
                           ue8m0=ue8m0, **args)
    assert torch.equal(s.cpu(), s_ref.cpu())
    assert torch.equal(q.view(torch.uint8).cpu(), q_ref.view(torch.uint8).cpu())


def test_paged_attention_noncausal_gathered_rows():
    case = _paged_case(20, 6, 128, 60)
    T = int(case["cu_q"][-1])
    # call B stacks reader rows of a larger packed chunk
    g = _gen(21)
    big = torch.randn(T + 50, 32, 128, generator=g).to(torch.bfloat16)
    rows = torch.randperm(T + 50, generator=g)[:T].sort().values
    big[rows] = case["q"]
    case_b = dict(case, q=big)
    got, lse, want, want_lse = _run_paged(case_b, causal=False, q_rows=rows)
    assert (got - want).abs().max().item() <= 2e-3
    assert torch.allclose(lse, want_lse, atol=2e-3, rtol=0)


def test_contiguous_causal_attention():
    g = _gen(30)
    lens = [1, 17, 64, 65, 200, 3]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int32)
    T = int(cu[-1])
    q = (torch.randn(T, 32, 128, generator=g) / math.sqrt(128)).to(torch.bfloat16)
    k = (torch.randn(T, 8, 128, generator=g) / math.sqrt(128)).to(torch.bfloat16)
    v = (torch.randn(T, 8, 128, generator=g) / math.sqrt(128)).to(torch.bfloat16)
    scale = 1 / math.sqrt(128)
    kv_len = torch.tensor(lens, dtype=torch.int32)
    out, lse = K.attention(q.to(DEV), cu.to(DEV), kv_len.to(DEV), n_queries=T,
                           max_q=max(lens), softmax_scale=scale, causal=True,
                           k_rows=k.to(DEV), v_rows=v.to(DEV), cu_k=cu.to(DEV),
                           n_kv=8, want_lse=True)
    want, want_lse = ref.varlen_attention(q, k, v, cu, scale, causal=True)
    assert (out.cpu().float() - want).abs().max().item() <= 2e-3
    assert torch.allclose(lse.cpu(), want_lse, atol=2e-3, rtol=0)


def test_merge_attn_quant():
    g = _gen(40)
    T, R, H, d = 57, 20, 32, 128
    a = torch.randn(T, H, d, generator=g).to(torch.bfloat16)
    b = torch.randn(R, H, d, generator=g).to(torch.bfloat16)
    la = torch.randn(H, T, generator=g) * 3
    lb = torch.randn(H, R, generator=g) * 3
    source = torch.full((T,), -1, dtype=torch.int32)
    source[torch.randperm(T, generator=g)[:R]] = torch.arange(R, dtype=torch.int32)
    q_ref, s_ref = ref.merge_attn_quant(a, la, b, lb, source)
    q, s = K.merge_attn_quant(a.to(DEV), la.to(DEV), b.to(DEV), lb.to(DEV), source.to(DEV))
    _check_quant(q, s, q_ref, s_ref, max_frac_off=1e-3, scale_rtol=0)


def test_qk_norm_rope_kv_equals_rope_then_scatter():
    """q, and the arena rows the fused kernel writes k and v into, are bit for
    bit qk_norm_rope followed by kv_row_scatter; 83 rows (a ragged last block
    of 16), arena rows in runs starting mid-page plus scattered singles, every
    other arena row untouched."""
    g = _gen(51)
    T, n_q, n_kv, d = 83, 32, 8, 128
    n_pages = 40
    qkv = torch.randn(T, (n_q + 2 * n_kv) * d, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, 4000, (T,), generator=g)
    cs = ref.rope_cache(4096, d, 1e6)
    qw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    run = torch.cat([torch.arange(9 * 16 + 5, 11 * 16), torch.arange(3 * 16, 4 * 16)])
    rest = torch.tensor([r for r in torch.randperm(n_pages * 16, generator=g).tolist()
                         if r not in set(run.tolist())][:T - run.numel()])
    row_dst = torch.cat([run, rest]).to(torch.int64)
    base_k = torch.randn(n_pages * 16, n_kv, d, generator=g).to(torch.bfloat16)
    base_v = torch.randn(n_pages * 16, n_kv, d, generator=g).to(torch.bfloat16)
    args = (qkv.to(DEV), pos.to(DEV), cs.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6, n_q, n_kv, d)
    q_a, k_a, v_a = K.qk_norm_rope(*args)
    kp_a = layout.k_pool_from_rows(base_k).to(DEV)
    vp_a = layout.v_pool_from_rows(base_v).to(DEV)
    K.kv_row_scatter(k_a.view(T, n_kv, d), v_a.view(T, n_kv, d), kp_a, vp_a,
                     torch.arange(T, device=DEV), row_dst.to(DEV))
    kp_b = layout.k_pool_from_rows(base_k).to(DEV)
    vp_b = layout.v_pool_from_rows(base_v).to(DEV)
    q_b = K.qk_norm_rope_kv(*args, kp_b, vp_b, row_dst.to(DEV))
    assert torch.equal(q_b.view(torch.int16), q_a.view(torch.int16))
    assert torch.equal(kp_b.view(torch.int16), kp_a.view(torch.int16))
    assert torch.equal(vp_b.view(torch.int16), vp_a.view(torch.int16))


def _qkv_rope_case(seed, M, n_q, n_kv, Kd, n_pages=0, ue8m0=False):
    """qkv GEMM operands (N(0,1) activations, N(0,0.02) weights, 1x128 and
    128x128 scales) plus the q/k norm + rotary inputs; positions include
    values past the cache, which the kernels clamp. With n_pages, distinct
    arena rows for every row: runs of consecutive slots that start mid-page,
    then scattered single rows."""
    g = _gen(seed)
    N, d = (n_q + 2 * n_kv) * 128, 128
    wq, ws = ref.quantize_weight_blocks(torch.randn(N, Kd, generator=g) * 0.02, ue8m0=ue8m0)
    xq, xs = ref.group_quant(torch.randn(M, Kd, generator=g), ue8m0=ue8m0)
    xs_dev = K.col_major_scales(M, Kd, DEV)
    xs_dev.copy_(xs)
    max_pos = 4096
    pos = torch.randint(0, max_pos + 64, (M,), generator=g)
    cs = ref.rope_cache(max_pos, d, 1e6)
    qw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    case = dict(gemm=(xq.to(DEV), xs_dev, wq.to(DEV), ws.to(DEV)),
                rope=(pos.to(DEV), cs.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6, n_q, n_kv))
    if n_pages:
        rows = n_pages * 16
        run = torch.cat([torch.arange(5 * 16 + 7, 5 * 16 + 7 + min(M, 300) // 2),
                         torch.arange(rows - min(M, 300) // 2, rows)])
        taken = set(run.tolist())
        rest = [r for r in torch.randperm(rows, generator=g).tolist() if r not in taken]
        case["row_dst"] = torch.cat([run, torch.tensor(rest[:M - run.numel()])]).to(torch.int64)
        case["base_k"] = torch.randn(rows, n_kv, d, generator=g).to(torch.bfloat16)
        case["base_v"] = torch.randn(rows, n_kv, d, generator=g).to(torch.bfloat16)
    return case


@pytest.mark.parametrize("M,n_q,n_kv,Kd,ue8m0", [(1, 32, 8, 2560, False), (517, 32, 8, 2560, False),
                                                 (4099, 32, 8, 2560, False), (300, 8, 2, 1024, False),
                                                 (700, 64, 8, 5120, False), (517, 32, 8, 2560, True)])
def test_fp8_gemm_qkv_rope_matches_gemm_then_norm_rope(M, n_q, n_kv, Kd, ue8m0):
    """The qkv GEMM with q/k norm + rotary in its epilogue equals fp8_gemm_nt
    followed by qk_norm_rope, bit for bit: q, k and v rows (ragged last tile,
    positions past the cache clamped, GQA 4:1 and 8:1, both scale modes)."""
    case = _qkv_rope_case(70 + M, M, n_q, n_kv, Kd, ue8m0=ue8m0)
    qkv = K.fp8_gemm_nt(*case["gemm"], ue8m0_scales=ue8m0)
    want = K.qk_norm_rope(qkv, *case["rope"], 128)
    got = K.fp8_gemm_qkv_rope(*case["gemm"], *case["rope"], ue8m0_scales=ue8m0)
    for name, x, y in zip("qkv", got, want):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16)), name


@pytest.mark.parametrize("M,n_q,n_kv,Kd", [(517, 32, 8, 2560), (2049, 64, 8, 5120)])
def test_fp8_gemm_qkv_rope_kv_matches_gemm_then_norm_rope_kv(M, n_q, n_kv, Kd):
    """With arena rows, the fused GEMM writes q and the K and V^T pages
    exactly as fp8_gemm_nt followed by qk_norm_rope_kv: every pool byte
    equal, the untouched rows included."""
    n_pages = (M + 15) // 16 + 40
    case = _qkv_rope_case(90 + M, M, n_q, n_kv, Kd, n_pages=n_pages)
    dst = case["row_dst"].to(DEV)
    pools = []
    for _ in range(2):
        pools.append((layout.k_pool_from_rows(case["base_k"]).to(DEV),
                      layout.v_pool_from_rows(case["base_v"]).to(DEV)))
    qkv = K.fp8_gemm_nt(*case["gemm"])
    q_a = K.qk_norm_rope_kv(qkv, *case["rope"], 128, *pools[0], dst)
    q_b = K.fp8_gemm_qkv_rope(*case["gemm"], *case["rope"], k_pool=pools[1][0],
                              v_pool=pools[1][1], row_dst=dst)
    assert torch.equal(q_b.view(torch.int16), q_a.view(torch.int16))
    assert torch.equal(pools[1][0].view(torch.int16), pools[0][0].view(torch.int16))
    assert torch.equal(pools[1][1].view(torch.int16), pools[0][1].view(torch.int16))


def test_kv_row_scatter_and_copy_bit_exact():
    g = _gen(50)
    n_pages, n_kv, d = 24, 8, 128
    rows = n_pages * 16
    k_pool_rows = torch.randn(rows, n_kv, d, generator=g).to(torch.bfloat16)
    v_pool_rows = torch.randn(rows, n_kv, d, generator=g).to(torch.bfloat16)
    T = 70
    k_src = torch.randn(T, n_kv, d, generator=g).to(torch.bfloat16)
    v_src = torch.randn(T, n_kv, d, generator=g).to(torch.bfloat16)
    src = torch.randperm(T, generator=g)[:50]
    dst = torch.randperm(rows, generator=g)[:50]
    kp = layout.k_pool_from_rows(k_pool_rows).to(DEV)
    vp = layout.v_pool_from_rows(v_pool_rows).to(DEV)
    K.kv_row_scatter(k_src.to(DEV), v_src.to(DEV), kp, vp, src.to(DEV), dst.to(DEV))
    ref.kv_row_scatter(k_pool_rows, v_pool_rows, k_src, v_src, src, dst)
    assert torch.equal(layout.k_rows(kp.cpu()), k_pool_rows)
    assert torch.equal(layout.v_rows(vp.cpu()), v_pool_rows)
    # runs of consecutive arena rows (a row's fresh tokens) starting mid-page,
    # in page order 9, 3, 17: the coalesced V^T writes of one page row
    run = torch.cat([torch.arange(9 * 16 + 5, 10 * 16), torch.arange(3 * 16, 4 * 16),
                     torch.arange(17 * 16, 17 * 16 + 9)])
    src2 = torch.randperm(T, generator=g)[:run.numel()]
    K.kv_row_scatter(k_src.to(DEV), v_src.to(DEV), kp, vp, src2.to(DEV), run.to(DEV))
    ref.kv_row_scatter(k_pool_rows, v_pool_rows, k_src, v_src, src2, run)
    assert torch.equal(layout.k_rows(kp.cpu()), k_pool_rows)
    assert torch.equal(layout.v_rows(vp.cpu()), v_pool_rows)
    # pool -> pool copy (tail of a kept page into a temporary)
    csrc = torch.randperm(rows, generator=g)[:30]
    cdst = torch.randperm(rows, generator=g)[:30]
    cdst = cdst[~torch.isin(cdst, csrc)]
    csrc = csrc[:cdst.numel()]
    K.kv_row_copy(kp, vp, csrc.to(DEV), cdst.to(DEV))
    k_pool_rows[cdst] = k_pool_rows[csrc]
    v_pool_rows[cdst] = v_pool_rows[csrc]
    assert torch.equal(layout.k_rows(kp.cpu()), k_pool_rows)
    assert torch.equal(layout.v_rows(vp.cpu()), v_pool_rows)


def test_gather_quant_rows_takes_rows_and_their_scales():
    """The fp8 row gather of the last layer's o_proj input: rows and their
    column-major 1x128 scales equal torch indexing, repeated rows included."""
    g = _gen(61)
    T, W = 333, 4096
    x = torch.randn(T, W, generator=g).to(torch.bfloat16).to(DEV)
    q, s = K.group_quant(x)
    idx = torch.tensor([0, 332, 17, 17, 200, 5], dtype=torch.int64)
    gq, gs = K.gather_quant_rows(q, s, idx.to(DEV))
    assert gs.stride() == (1, idx.numel())
    assert torch.equal(gq.cpu().view(torch.uint8), q.cpu().view(torch.uint8)[idx])
    assert torch.equal(gs.cpu(), s.cpu()[idx])
    eq, es = K.gather_quant_rows(q, s, torch.empty(0, dtype=torch.int64, device=DEV))
    assert eq.shape == (0, W) and es.shape == (0, W // 128)


def test_gather_final_norm_and_answer_bits():
    g = _gen(60)
    T, H = 90, 2560
    table = torch.randn(500, H, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 500, (T,), generator=g)
    assert torch.equal(K.gather_rows(table.to(DEV), idx.to(DEV)).cpu(), table[idx])
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    resid = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    fin = torch.tensor([3, 17, 89, 0], dtype=torch.int64)
    want, _ = ref.fused_add_rms_norm(hidden[fin], resid[fin], w, 1e-6)
    got = K.final_norm(hidden.to(DEV), resid.to(DEV), fin.to(DEV), w.to(DEV), 1e-6).cpu()
    diff = (got.float() - want.float()).abs()
    assert (diff <= want.float().abs() * 2 ** -7).all()
    # readout: 6 retained rows, TRUE = the first three
    w_ans = (torch.randn(6, H, generator=g) * 0.05).to(torch.bfloat16)
    is_true = torch.tensor([1, 1, 1, 0, 0, 0], dtype=torch.uint8)
    normed = torch.randn(64, H, generator=g).to(torch.bfloat16)
    bits_ref, margin_ref = ref.answer_bits(normed, w_ans, [0, 1, 2], [3, 4, 5])
    bits, margin = K.answer_bits(normed.to(DEV), w_ans.to(DEV), is_true.to(DEV))
    clear = margin_ref.abs() > 0.05
    assert torch.equal(bits.cpu()[clear], bits_ref[clear])
    assert (margin.cpu() - margin_ref).abs().max().item() < 0.1
    # AnswerRows.logits: the per-class maxima of the same bf16 scores
    best_t, best_f = K.answer_logits(normed.to(DEV), w_ans.to(DEV), is_true.to(DEV))
    assert best_t.dtype == torch.bfloat16 and best_t.shape == (64,)
    assert torch.equal((best_t > best_f).to(torch.uint8).cpu(), bits.cpu())
    assert torch.equal((best_t.float() - best_f.float()).cpu(), margin.cpu())
    scores = normed.float() @ w_ans.float().t()
    for got, cols in ((best_t, [0, 1, 2]), (best_f, [3, 4, 5])):
        want = scores[:, cols].amax(dim=1)
        assert ((got.cpu().float() - want).abs() <= want.abs() * 2 ** -7 + 1e-3).all()


# The two tree kernels: "stream" (qh_tree_attention, node pages streamed
# per q-tile) and "node" (qh_tree_attention_resident, node K/V held in LDS;
# page-table rows of at most 16 pages).
TREE_KERNELS = ["node", "stream"]


def _tree_case(seed, *, n_nodes=3, segs=9, n_q=32, n_kv=8, d=128, nan_unread=True, sd=None,
               kernel="stream", seg_len=(1, 140), node_len=None):
    """Chunk rows in causal segments; some segments read one of n_nodes
    resident nodes (random lengths, partial last pages, permuted physical
    pages); every arena row no node reads is NaN. Q, K, V ~ N(0, sd^2),
    sd = 1/sqrt(d) by default (the C1 distribution). kernel "node" keeps
    the nodes within 256 keys and the table 16 pages wide."""
    sd = 1 / math.sqrt(d) if sd is None else sd
    g = _gen(seed)
    page = 16
    top = 257 if kernel == "node" else 300
    if node_len is None:
        node_len = [int(x) for x in torch.randint(1, top, (n_nodes,), generator=g)]
    n_nodes = len(node_len)
    widths = [-(-n // page) for n in node_len]
    n_pages = sum(widths) + 5
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    width = 16 if kernel == "node" else max(widths)
    assert max(widths) <= width
    table = torch.zeros(n_nodes, width, dtype=torch.int32)
    at = 0
    for i, w in enumerate(widths):
        table[i, :w] = perm[at:at + w]
        at += w
    lens = [int(x) for x in torch.randint(seg_len[0], seg_len[1], (segs,), generator=g)]
    lens[0] = 1
    cu_a = [0]
    for n in lens:
        cu_a.append(cu_a[-1] + n)
    seg_read = torch.tensor([int(torch.randint(-1, n_nodes, (1,), generator=g)) for _ in lens],
                            dtype=torch.int32)
    T = cu_a[-1]
    q = (torch.randn(T, n_q, d, generator=g) * sd).to(torch.bfloat16)
    k3 = (torch.randn(T, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    v3 = (torch.randn(T, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    k_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    v_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    if nan_unread:
        read = torch.zeros(n_pages * page, dtype=torch.bool)
        for i, n in enumerate(node_len):
            for j in range(n):
                read[int(table[i, j // page]) * page + j % page] = True
        k_rows[~read] = float("nan")
        v_rows[~read] = float("nan")
    return dict(q=q, k3=k3, v3=v3, k_rows=k_rows, v_rows=v_rows, table=table,
                used=torch.tensor(node_len, dtype=torch.int32), cu_a=torch.tensor(cu_a, dtype=torch.int32),
                seg_read=seg_read, T=T, kernel=kernel)


def _run_tree(case, fp8, ue8m0=False):
    kp = layout.k_pool_from_rows(case["k_rows"]).to(DEV)
    vp = layout.v_pool_from_rows(case["v_rows"]).to(DEV)
    return K.tree_attention(case["q"].to(DEV), case["k3"].to(DEV), case["v3"].to(DEV),
                            case["cu_a"].to(DEV), case["seg_read"].to(DEV),
                            softmax_scale=1 / math.sqrt(128), k_pool=kp, v_pool=vp,
                            table=case["table"].to(DEV), used=case["used"].to(DEV), fp8=fp8,
                            ue8m0=ue8m0, resident=case["kernel"] == "node")


@pytest.mark.parametrize("kernel", TREE_KERNELS)
@pytest.mark.parametrize("seed,n_kv", [(60, 8), (61, 8), (62, 4)])
def test_tree_attention_matches_the_oracle(seed, n_kv, kernel):
    """The fused tree kernels (node keys, then own rows, one softmax) within
    max-abs 2e-3 of the fp32 oracle; unread arena rows are NaN."""
    case = _tree_case(seed, n_kv=n_kv, kernel=kernel)
    got = _run_tree(case, fp8=False).float().cpu()
    want = ref.tree_attention(case["q"], case["k3"], case["v3"], case["cu_a"], case["seg_read"],
                              case["k_rows"], case["v_rows"], case["table"], case["used"],
                              1 / math.sqrt(128))
    assert torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    assert err <= 2e-3, f"max-abs {err}"


def _tree_rounded_reference(case, scale):
    """The oracle's attention with the kernel's two roundings: the
    unnormalized probabilities (<= 1) to bf16 for the P.V product (the sum
    l stays fp32), and the output to bf16."""
    cu = case["cu_a"].tolist()
    T, H, d = case["q"].shape
    out = torch.zeros(T, H, d)
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        c, r = b - a, int(case["seg_read"][s])
        k, v = case["k3"][a:b].float(), case["v3"][a:b].float()
        vis = ref.causal_visible(c, c)
        if r >= 0:
            n = int(case["used"][r])
            k = torch.cat([ref.gather_pages(case["k_rows"], case["table"][r], n).float(), k])
            v = torch.cat([ref.gather_pages(case["v_rows"], case["table"][r], n).float(), v])
            vis = torch.cat([torch.ones(c, n, dtype=torch.bool), vis], 1)
        kk = k.repeat_interleave(H // k.shape[1], 1)
        vv = v.repeat_interleave(H // v.shape[1], 1)
        sc = torch.einsum("chd,lhd->hcl", case["q"][a:b].float(), kk) * scale
        sc = sc.masked_fill(~vis[None], float("-inf"))
        p = torch.exp(sc - sc.amax(-1, keepdim=True))
        l = p.sum(-1, keepdim=True)
        o = torch.einsum("hcl,lhd->chd", p.to(torch.bfloat16).float() / l, vv)
        out[a:b] = o.to(torch.bfloat16).float()
    return out


@pytest.mark.parametrize("kernel", TREE_KERNELS)
def test_tree_attention_sharp_softmax_matches_its_rounding_model(kernel):
    """Q, K, V ~ N(0, 1): peaked probabilities that expose any mismatch of a
    probability with the wrong key's V. Against the oracle with the kernel's
    bf16 roundings applied: within one bf16 step of the output (2^-7
    relative; the kernel rounds probabilities against the running maximum,
    the model against the final one) plus 2e-3."""
    case = _tree_case(65, sd=1.0, kernel=kernel)
    got = _run_tree(case, fp8=False).float().cpu()
    want = _tree_rounded_reference(case, 1 / math.sqrt(128))
    excess = ((got - want).abs() - (2.0 ** -7 * want.abs() + 2e-3)).max().item()
    assert excess <= 0, f"beyond one bf16 step by {excess}"


@pytest.mark.parametrize("kernel", TREE_KERNELS)
def test_tree_attention_is_deterministic(kernel):
    case = _tree_case(66, sd=1.0, kernel=kernel)
    first = _run_tree(case, fp8=False).cpu()
    for _ in range(3):
        assert torch.equal(_run_tree(case, fp8=False).cpu(), first)


@pytest.mark.parametrize("kernel", TREE_KERNELS)
def test_tree_attention_at_64_query_heads(kernel):
    """Qwen3-32B heads (64 query / 8 KV, 16 head groups: two workgroups'
    head groups per KV head) within max-abs 2e-3 of the fp32 oracle."""
    case = _tree_case(69, n_q=64, n_kv=8, segs=12, kernel=kernel)
    got = _run_tree(case, fp8=False).float().cpu()
    want = ref.tree_attention(case["q"], case["k3"], case["v3"], case["cu_a"], case["seg_read"],
                              case["k_rows"], case["v_rows"], case["table"], case["used"],
                              1 / math.sqrt(128))
    assert torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    assert err <= 2e-3, f"max-abs {err}"


def test_node_resident_tree_attention_with_interleaved_nodes():
    """60 segments reading 4 nodes (and none) in random order: every
    workgroup of the node-resident kernel walks several q-tiles and reloads
    its node whenever the next q-tile reads another one. Within max-abs 2e-3
    of the fp32 oracle; unread arena rows are NaN."""
    case = _tree_case(67, n_nodes=4, segs=60, seg_len=(1, 200), kernel="node")
    got = _run_tree(case, fp8=False).float().cpu()
    want = ref.tree_attention(case["q"], case["k3"], case["v3"], case["cu_a"], case["seg_read"],
                              case["k_rows"], case["v_rows"], case["table"], case["used"],
                              1 / math.sqrt(128))
    assert torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    assert err <= 2e-3, f"max-abs {err}"


def test_node_resident_tree_attention_at_the_prefix_shared_layer_shape():
    """The prefix-shared layer: 64 segments of 32-256 rows all reading one
    256-key node (16 whole pages), 32 query / 8 KV heads; the fp8 output and
    scales bit-identical to the streaming kernel's on the same inputs (the
    same arithmetic in the same key order), and the bf16 output within
    max-abs 2e-3 of the fp32 oracle run on the GPU."""
    case = _tree_case(68, n_nodes=1, segs=64, seg_len=(32, 257), kernel="node",
                      node_len=[256])
    case["seg_read"].zero_()
    got = _run_tree(case, fp8=False).float()
    with torch.no_grad():
        want = ref.tree_attention(case["q"].to(DEV), case["k3"].to(DEV), case["v3"].to(DEV),
                                  case["cu_a"], case["seg_read"], case["k_rows"].to(DEV),
                                  case["v_rows"].to(DEV), case["table"], case["used"],
                                  1 / math.sqrt(128))
    err = (got - want.to(got.device)).abs().max().item()
    assert err <= 2e-3, f"max-abs {err}"
    q1, s1 = _run_tree(case, fp8=True)
    q2, s2 = _run_tree(dict(case, kernel="stream"), fp8=True)
    assert torch.equal(s1.cpu(), s2.cpu())
    assert torch.equal(q1.view(torch.uint8).cpu(), q2.view(torch.uint8).cpu())


@pytest.mark.parametrize("kernel", TREE_KERNELS)
@pytest.mark.parametrize("ue8m0", [False, True])
def test_tree_attention_fp8_matches_quantized_bf16(ue8m0, kernel):
    case = _tree_case(63, kernel=kernel)
    out = _run_tree(case, fp8=False)
    q_ref, s_ref = K.group_quant(out.view(case["T"], -1), ue8m0)
    q, s = _run_tree(case, fp8=True, ue8m0=ue8m0)
    assert torch.equal(s.cpu(), s_ref.cpu())
    assert torch.equal(q.view(torch.uint8).cpu(), q_ref.view(torch.uint8).cpu())


def test_tree_attention_agrees_with_the_two_pass_form():
    """Call A + call B + merge_attn_quant (the reference's three launches,
    with their bf16 roundings) against the fused kernel. The merge's bf16
    weights and bf16 partial outputs move values by ~0.4% relative, which
    after two 1x128 quantizations (on slightly different grids) leaves the
    CPU oracle's own two forms 1.6% apart in relative L2 with 2.2% of values
    beyond one e4m3 step; the bars are 3% and 5%."""
    case = _tree_case(64, nan_unread=False)
    T = case["T"]
    kp = layout.k_pool_from_rows(case["k_rows"]).to(DEV)
    vp = layout.v_pool_from_rows(case["v_rows"]).to(DEV)
    q3, k3, v3 = case["q"].to(DEV), case["k3"].to(DEV), case["v3"].to(DEV)
    cu_a = case["cu_a"].to(DEV)
    scale = 1 / math.sqrt(128)
    a_len = cu_a[1:] - cu_a[:-1]
    out_a, lse_a = K.attention(q3, cu_a, a_len.to(torch.int32), n_queries=T,
                               max_q=int(a_len.max()), softmax_scale=scale, causal=True,
                               k_rows=k3, v_rows=v3, cu_k=cu_a, n_kv=8, want_lse=True)
    # call B: the readers of each node stacked into one sequence per node
    sr = case["seg_read"]
    rows, cu_q, used, tab = [], [0], [], []
    for r in range(case["table"].shape[0]):
        mine = [torch.arange(int(case["cu_a"][s]), int(case["cu_a"][s + 1]))
                for s in range(len(sr)) if int(sr[s]) == r]
        if not mine:
            continue
        rows.append(torch.cat(mine))
        cu_q.append(cu_q[-1] + rows[-1].numel())
        used.append(int(case["used"][r]))
        tab.append(case["table"][r])
    rows = torch.cat(rows)
    source = torch.full((T,), -1, dtype=torch.int32)
    source[rows] = torch.arange(rows.numel(), dtype=torch.int32)
    out_b, lse_b = K.attention(q3, torch.tensor(cu_q, dtype=torch.int32, device=DEV),
                               torch.tensor(used, dtype=torch.int32, device=DEV),
                               n_queries=rows.numel(), max_q=max(cu_q[i + 1] - cu_q[i] for i in range(len(used))),
                               softmax_scale=scale, causal=False, k_pool=kp, v_pool=vp,
                               table=torch.stack(tab).to(DEV), q_rows=rows.to(DEV), n_kv=8,
                               want_lse=True)
    q2, s2 = K.merge_attn_quant(out_a, lse_a, out_b, lse_b, source.to(DEV))
    q1, s1 = _run_tree(case, fp8=True)
    two = ref.dequant_rows(q2.cpu(), s2.cpu())
    one = ref.dequant_rows(q1.cpu(), s1.cpu())
    # the bf16 intermediates of the two-pass form move a value by ~2^-8
    # relative, which can flip its e4m3 rounding by one step (2^-3 relative)
    rel = ((two - one).norm() / one.norm()).item()
    assert rel < 0.03, f"relative L2 {rel}"
    # one e4m3 step at each value, in units of its group's scale: 2^(e-3)
    # for normal values (e = floor(log2 |x|)), 2^-9 below 2^-6
    scale = torch.maximum(s1.cpu(), s2.cpu()).repeat_interleave(128, dim=1)
    mag = torch.maximum(two.abs(), one.abs()) / scale
    step = torch.where(mag >= 2.0 ** -6, torch.exp2(torch.floor(torch.log2(mag.clamp(min=1e-30))) - 3),
                       torch.full_like(mag, 2.0 ** -9)) * scale
    beyond = ((two - one).abs() > step * 1.001).float().mean().item()
    assert beyond < 0.05, f"values off by more than one e4m3 step: {beyond}"


def test_every_entry_point_takes_empty_inputs():
    """Zero rows (an empty chunk, no answer rows, no reads) through every
    entry point: each returns empty outputs of the right shapes and launches
    nothing; the sizes check before the pointers, since an empty tensor's
    storage may be null."""
    bf, f8 = torch.bfloat16, torch.float8_e4m3fn
    H, n_q, n_kv, d = 2560, 32, 8, 128
    e_bf = torch.empty(0, H, dtype=bf, device=DEV)
    w = torch.ones(H, dtype=bf, device=DEV)
    q, s = K.add_rmsnorm_quant(e_bf, w, 1e-6)
    assert q.shape == (0, H) and s.shape == (0, H // 128)
    q, s = K.add_rmsnorm_quant(e_bf, w, 1e-6, residual=torch.empty(0, H, dtype=bf, device=DEV))
    assert q.shape == (0, H)
    q, s = K.group_quant(e_bf)
    assert q.shape == (0, H) and s.shape == (0, H // 128)
    q, s = K.silu_mul_quant(torch.empty(0, 2 * H, dtype=bf, device=DEV))
    assert q.shape == (0, H)
    # GEMMs with no rows
    a = torch.empty(0, H, dtype=f8, device=DEV)
    a_s = K.col_major_scales(0, H, DEV)
    wq = torch.zeros(512, H, dtype=f8, device=DEV)
    ws = torch.ones(4, H // 128, dtype=torch.float32, device=DEV)
    assert K.fp8_gemm_nt(a, a_s, wq, ws).shape == (0, 512)
    q, s = K.fp8_gemm_silu_quant(a, a_s, wq, ws)
    assert q.shape == (0, 256) and s.shape == (0, 2)
    wqkv = torch.zeros((n_q + 2 * n_kv) * d, H, dtype=f8, device=DEV)
    wqkv_s = torch.ones((n_q + 2 * n_kv), H // 128, dtype=torch.float32, device=DEV)
    cos_sin = torch.zeros(64, d, dtype=bf, device=DEV)
    hw = torch.ones(d, dtype=bf, device=DEV)
    pos = torch.empty(0, dtype=torch.int64, device=DEV)
    qq, kk, vv = K.fp8_gemm_qkv_rope(a, a_s, wqkv, wqkv_s, pos, cos_sin, hw, hw, 1e-6, n_q, n_kv)
    assert qq.shape == (0, n_q * d) and kk.shape == vv.shape == (0, n_kv * d)
    kp = torch.zeros(4, n_kv, 16, d, dtype=bf, device=DEV)
    vp = torch.zeros(4, n_kv, d, 16, dtype=bf, device=DEV)
    qq = K.fp8_gemm_qkv_rope(a, a_s, wqkv, wqkv_s, pos, cos_sin, hw, hw, 1e-6, n_q, n_kv,
                             k_pool=kp, v_pool=vp, row_dst=pos)
    assert qq.shape == (0, n_q * d) and not kp.any() and not vp.any()
    qkv = torch.empty(0, (n_q + 2 * n_kv) * d, dtype=bf, device=DEV)
    qq, kk, vv = K.qk_norm_rope(qkv, pos, cos_sin, hw, hw, 1e-6, n_q, n_kv, d)
    assert qq.shape == (0, n_q * d)
    assert K.qk_norm_rope_kv(qkv, pos, cos_sin, hw, hw, 1e-6, n_q, n_kv, d, kp, vp,
                             pos).shape == (0, n_q * d)
    # KV movement with nothing to move
    rows = torch.empty(0, n_kv, d, dtype=bf, device=DEV)
    K.kv_row_scatter(rows, rows, kp, vp, pos, pos)
    K.kv_row_copy(kp, vp, pos, pos)
    assert not kp.any() and not vp.any()
    # attention over no sequences, and over sequences with no query rows
    q3 = torch.empty(0, n_q, d, dtype=bf, device=DEV)
    table = torch.zeros(2, 4, dtype=torch.int32, device=DEV)
    used = torch.tensor([16, 32], dtype=torch.int32, device=DEV)
    for cu in (torch.zeros(1, dtype=torch.int32, device=DEV),
               torch.zeros(3, dtype=torch.int32, device=DEV)):
        n_seqs = cu.numel() - 1
        out, lse = K.attention(q3, cu, used[:n_seqs], n_queries=0, max_q=0, softmax_scale=0.1,
                               causal=True, k_pool=kp, v_pool=vp, table=table[:max(n_seqs, 1)],
                               n_kv=n_kv, want_lse=True)
        assert out.shape == (0, n_q, d) and lse.shape == (n_q, 0)
        q8, s8 = K.attention_fp8(q3, cu, used[:n_seqs], n_queries=0, max_q=0,
                                 softmax_scale=0.1, causal=True, k_pool=kp, v_pool=vp,
                                 table=table[:max(n_seqs, 1)], n_kv=n_kv)
        assert q8.shape == (0, n_q * d) and s8.shape == (0, n_q)
    for resident in (False, True):
        q8, s8 = K.tree_attention(q3, rows, rows, torch.zeros(1, dtype=torch.int32, device=DEV),
                                  torch.empty(0, dtype=torch.int32, device=DEV),
                                  softmax_scale=0.1, k_pool=kp, v_pool=vp, table=table,
                                  used=used, resident=resident)
        assert q8.shape == (0, n_q * d) and s8.shape == (0, n_q)
    lse0 = torch.empty(n_q, 0, dtype=torch.float32, device=DEV)
    q8, s8 = K.merge_attn_quant(q3, lse0, q3, lse0, torch.empty(0, dtype=torch.int32,
                                                                device=DEV))
    assert q8.shape == (0, n_q * d)
    # row gathers, norms and the readout with no rows
    idx = torch.empty(0, dtype=torch.int64, device=DEV)
    table_rows = torch.ones(10, H, dtype=bf, device=DEV)
    assert K.gather_rows(table_rows, idx).shape == (0, H)
    full = torch.ones(5, H, dtype=bf, device=DEV)
    assert K.final_norm(full, full.clone(), idx, w, 1e-6).shape == (0, H)
    hid, res = K.fused_add_rms_norm(e_bf.clone(), e_bf.clone(), w, 1e-6)
    assert hid.shape == res.shape == (0, H)
    w_ans = torch.ones(4, H, dtype=bf, device=DEV)
    is_true = torch.tensor([1, 1, 0, 0], dtype=torch.uint8, device=DEV)
    bits, margin = K.answer_bits(e_bf, w_ans, is_true)
    assert bits.shape == margin.shape == (0,)
    t, f = K.answer_logits(e_bf, w_ans, is_true)
    assert t.shape == f.shape == (0,)
    assert K.e4m3_encode(torch.empty(0, dtype=torch.float32, device=DEV)).shape == (0,)
    torch.cuda.synchronize()
