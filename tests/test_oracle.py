"""Pin the CPU oracle: known answers, closed forms, independent restatements, brute force.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong rounding mode, a transposed operand, a reordered product) fails.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8_spec
from oracle import quant_ref as R
from tests._util import gen, rand_i8, rel_err


# ---------------------------------------------------------------- quantize_rows / weight (int8)
def test_known_answer_per_channel_weight():
    # reference tests/test_quant.py:43-50
    w = torch.ones(16, 32)
    w[0] *= 100.0
    q, s = R.quantize_weight(w, "int8")
    assert q.dtype == torch.int8 and s.shape == (16,)
    assert torch.all(q == 127)
    assert float(s[0]) == pytest.approx(100.0 / 127)
    assert float(s[1]) == pytest.approx(1.0 / 127)


def test_zero_row_quantizes_to_zero():
    # reference tests/test_quant.py:34-40: padded rows stay exactly zero
    x = torch.zeros(2, 64)
    for mode in ("int8", "fp8"):
        q, s = R.quantize_rows(x, mode)
        assert torch.all(q.float() == 0)
        assert torch.all(s == torch.tensor(1e-12, dtype=torch.float32) / (127.0 if mode == "int8" else 448.0))


def test_round_half_even_and_symmetric_clamp():
    # amax 127 -> scale exactly 1: x.5 values round to even, -amax maps to -127 (never -128)
    x = torch.tensor([[127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -127.0]])
    q, s = R.quantize_rows(x, "int8")
    assert float(s) == 1.0
    assert q.tolist() == [[127, 2, 4, -2, -4, 0, 0, 2, 126, -127]]


def test_int8_quant_matches_numpy_float32_restatement():
    g = gen(1)
    x = R.outlier_activations(g, 64, 1000).float()
    xn = x.numpy().astype(np.float32)
    amax = np.maximum(np.abs(xn).max(axis=1, keepdims=True), np.float32(1e-12))
    scale = (amax / np.float32(127.0)).astype(np.float32)
    qn = np.clip(np.rint((xn / scale).astype(np.float32)), -127, 127).astype(np.int8)
    q, s = R.quantize_rows(x, "int8")
    assert np.array_equal(q.numpy(), qn)
    assert np.array_equal(s.numpy(), scale)


def test_int8_quant_is_nearest_integer_bruteforce():
    # every q is the integer in [-127, 127] nearest to the fp32 quotient (ties to even)
    g = gen(2)
    x = torch.randn(8, 40, generator=g)
    q, s = R.quantize_rows(x, "int8")
    quot = (x / s).double()
    cand = torch.arange(-127, 128, dtype=torch.float64)
    for r in range(8):
        for c in range(40):
            d = (cand - quot[r, c]).abs()
            best = cand[d == d.min()]
            want = best[0] if len(best) == 1 else best[(best % 2) == 0][0]
            assert int(q[r, c]) == int(want)


# ---------------------------------------------------------------- quantize_rows_with_amax
@pytest.mark.parametrize("mode", ["int8", "fp8"])
def test_with_amax_equals_quantize_rows_at_the_row_max(mode):
    # given the row's own max |x| it is quantize_rows (pinned above) bit for bit; a dropped floor,
    # a swapped 127 / 448 or a missing division differs on these rows
    g = gen(3)
    x = R.outlier_activations(g, 24, 520).float()
    x[3] = 0.0  # the 1e-12 floor
    x[5, 7] = 1e-30  # a denormal-free tiny row amax
    x[5, :7] = 0.0
    x[5, 8:] = 0.0
    q_ref, s_ref = R.quantize_rows(x, mode)
    q, s = R.quantize_rows_with_amax(x, x.abs().amax(dim=1), mode)
    assert torch.equal(s, s_ref)
    assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))


def test_with_amax_known_answers_and_clamp():
    # amax above the row max: scale amax / 127 = 1 exactly, so q = round_half_even(x)
    x = torch.tensor([[1.0, -0.5, 2.5, 3.5], [100.0, 3.0, -100.0, 0.0]])
    q, s = R.quantize_rows_with_amax(x[:1], torch.tensor([127.0]), "int8")
    assert float(s) == 1.0 and q.tolist() == [[1, 0, 2, 4]]
    # amax below the row max: quotients beyond 127 clamp symmetrically (never -128)
    q, s = R.quantize_rows_with_amax(x[1:], torch.tensor([50.0]), "int8")
    assert float(s) == np.float32(50.0) / np.float32(127.0)
    quot = (x[1:] / s).tolist()[0]
    assert q.tolist() == [[127, round(quot[1]), -127, 0]]
    # fp8: scale amax / 448, quotient clamped to +-448 before the cast
    q, s = R.quantize_rows_with_amax(torch.tensor([[1000.0, -1000.0, 2.0]]), torch.tensor([448.0]), "fp8")
    assert float(s) == 1.0 and q.float().tolist() == [[448.0, -448.0, 2.0]]


def test_with_amax_keeps_a_nan_amax():
    # torch's clamp_min keeps NaN: a NaN row amax gives a NaN scale, as quantize_rows gives for a NaN row
    x = torch.tensor([[1.0, float("nan"), 2.0]])
    _, s_ref = R.quantize_rows(x, "int8")
    _, s = R.quantize_rows_with_amax(x, torch.tensor([float("nan")]), "int8")
    assert torch.isnan(s_ref).all() and torch.isnan(s).all()


# ---------------------------------------------------------------- FP8 (OCP E4M3)
def test_torch_e4m3fn_cast_matches_spec_encoder():
    # every finite code, every midpoint, neighbours of both, and a dense sweep of fp32 bit patterns
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8_spec.decode(codes)
    fin = np.unique(vals[np.isfinite(vals)])
    mids = (fin[1:] + fin[:-1]) / 2
    base = np.concatenate([fin, mids]).astype(np.float32)
    nb = base.view(np.int32)
    sweep = np.arange(0, 0x43E00000, 997, dtype=np.int64).astype(np.int32).view(np.float32)  # [0, 448]
    x = np.concatenate([base, (nb + 1).view(np.float32), (nb - 1).view(np.float32), sweep])
    x = np.concatenate([x, -x])
    x = x[np.isfinite(x) & (np.abs(x) <= 448)].astype(np.float32)
    ours = fp8_spec.encode(x)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)


def test_fp8_spec_decode_known_values():
    assert fp8_spec.decode(np.array([0x7E]))[0] == 448.0
    assert fp8_spec.decode(np.array([0x01]))[0] == 2.0 ** -9
    assert fp8_spec.decode(np.array([0x38]))[0] == 1.0
    assert np.isnan(fp8_spec.decode(np.array([0x7F]))[0])


def test_fp8_quant_rows_clamps_and_scales():
    x = torch.tensor([[448.0, -448.0, 1.0, 0.0], [1.0, 2.0, 4.0, -8.0]])
    q, s = R.quantize_rows(x, "fp8")
    assert torch.equal(s.reshape(-1), torch.tensor([1.0, 8.0 / 448.0]))
    qf = q.float()
    assert qf[0].tolist() == [448.0, -448.0, 1.0, 0.0]
    assert float(qf[1, 3]) == -448.0


# ---------------------------------------------------------------- accumulation
def test_bruteforce_handworked_and_transpose_detector():
    a = torch.tensor([[1, 2, 3, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0]], dtype=torch.int8)
    w = torch.zeros(2, 16, dtype=torch.int8)
    w[0, :3] = torch.tensor([4, 5, 6], dtype=torch.int8)
    w[1, 0] = -7
    out = R.int_accumulate_bruteforce(a, w)
    assert out.tolist() == [[1 * 4 + 2 * 5 + 3 * 6, -7]]
    # non-square, non-symmetric: a transposed operand cannot produce the same shape/values
    g = gen(3)
    A, Wt = rand_i8(g, 5, 32), rand_i8(g, 3, 32)
    ref = [[sum(int(A[m, k]) * int(Wt[n, k]) for k in range(32)) for n in range(3)] for m in range(5)]
    assert R.int_accumulate_bruteforce(A, Wt).tolist() == ref


def test_int_accumulate_float64_equals_bruteforce_at_extremes():
    # all-127 rows at K = 12288 reach 127*127*12288 = 1.98e8 (> 2**24, where fp32 would round)
    Kd = 12288
    a = torch.full((3, Kd), 127, dtype=torch.int8)
    a[1] = -127
    w = torch.full((2, Kd), 127, dtype=torch.int8)
    exact = R.int_accumulate_bruteforce(a, w)
    assert int(exact[0, 0]) == 127 * 127 * Kd
    assert torch.equal(R.int_accumulate(a, w), exact)
    g = gen(4)
    A, Wt = rand_i8(g, 40, 4096), rand_i8(g, 24, 4096)
    assert torch.equal(R.int_accumulate(A, Wt), R.int_accumulate_bruteforce(A, Wt))


def test_fp32_emulation_agrees_below_2_24():
    # the reference's own accumulator (quant.py:161) is exact while partial sums stay < 2**24
    g = gen(5)
    A, Wt = rand_i8(g, 16, 1024), rand_i8(g, 8, 1024)
    assert torch.equal(R.fp32_accumulate(A, Wt).to(torch.int64), R.int_accumulate_bruteforce(A, Wt))


# ---------------------------------------------------------------- dequant
def test_dequant_known_answer_all_ones():
    # x = 1, W = 1: q = 127, scales 1/127 -> (127*127*K * (1/127)) * (1/127) == K exactly in bf16
    Kd = 256
    x = torch.ones(2, Kd)
    w = torch.ones(4, Kd)
    wq, ws = R.quantize_weight(w, "int8")
    out, acc, q, s = R.int8_linear(x, wq, ws, torch.bfloat16)
    assert torch.all(acc == 127 * 127 * Kd)
    assert torch.all(out.float() == Kd)


def test_dequant_order_matches_numpy_left_to_right():
    g = gen(6)
    acc = torch.randint(-2**20, 2**20, (32, 48), generator=g)
    st = torch.rand(32, 1, generator=g) * 1e-2
    sc = torch.rand(48, generator=g) * 1e-3
    ours = R.dequant(acc, st, sc, torch.float32).numpy()
    a = acc.numpy().astype(np.float32)
    want = (a * st.numpy().astype(np.float32)).astype(np.float32) * sc.numpy().astype(np.float32)[None, :]
    assert np.array_equal(ours, want.astype(np.float32))
    # and it differs from the pre-multiplied form somewhere (so the order is actually pinned)
    pre = a * (st.numpy() * sc.numpy()[None, :]).astype(np.float32)
    assert not np.array_equal(ours, pre.astype(np.float32))


# ---------------------------------------------------------------- whole-linear behaviour
@pytest.mark.parametrize("mode,limit", [("fp8", 0.06), ("int8", 0.02)])
def test_linear_error_bounds_of_reference_tests(mode, limit):
    # reference tests/test_quant.py:15-26, applied to the oracle's forward
    torch.manual_seed(0)
    weight = torch.randn(96, 256) * 0.02
    x = torch.randn(3, 5, 256, dtype=torch.bfloat16)
    wq, ws = R.quantize_weight(weight.to(torch.bfloat16), mode)
    out = R.linear_forward(x, wq, ws, mode, torch.bfloat16)
    assert out.shape == (3, 5, 96) and out.dtype == torch.bfloat16
    assert rel_err(out, x.float() @ weight.t()) < limit
    emu = R.emulated_linear(x.reshape(-1, 256), wq, ws, mode, torch.bfloat16)
    assert rel_err(out.reshape(-1, 96), emu) < 1e-2


def test_outlier_rows_do_not_crush_other_rows():
    # reference tests/test_quant.py:29-40
    torch.manual_seed(0)
    weight = torch.randn(32, 64)
    x = torch.randn(4, 64)
    x[1] *= 1000.0
    x[3] = 0.0
    wq, ws = R.quantize_weight(weight, "int8")
    out = R.linear_forward(x, wq, ws, "int8", torch.float32)
    ref = x @ weight.t()
    assert rel_err(out[0], ref[0]) < 0.02
    assert torch.all(out[3] == 0)


# ---------------------------------------------------------------- norm and SwiGLU
def test_rmsnorm_matches_transformers_qwen3_5():
    mod = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    g = gen(7)
    H = 512
    x = R.outlier_activations(g, 16, H)
    w = (0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    norm = mod.Qwen3_5RMSNorm(H, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w.float())
        want = norm(x)
    assert torch.equal(R.rmsnorm(x, w, 1e-6, zero_centered=True), want)


def test_swiglu_closed_form_and_halves():
    g = gen(8)
    gu = (torch.randn(6, 64, generator=g) * 3).to(torch.bfloat16)
    h = R.swiglu(gu)
    gate, up = gu[:, :32].double(), gu[:, 32:].double()
    exact = gate / (1 + torch.exp(-gate)) * up
    assert h.shape == (6, 32)
    # two bf16 roundings: within 2**-7 relative of the exact value
    assert torch.all((h.double() - exact).abs() <= exact.abs() * 2.0 ** -7 + 1e-6)
    swapped = R.swiglu(torch.cat([gu[:, 32:], gu[:, :32]], dim=1))
    assert not torch.equal(h, swapped)


def test_gated_input_known_answers_and_closed_form():
    """core.py:297, out * sigmoid(gate): sigmoid(0) = 1/2 exactly, saturation at |gate| = 30, and the
    float64 closed form within two bf16 roundings (sigmoid rounded, then the product)."""
    g = gen(21)
    out = (torch.randn(5, 96, generator=g) * 4).to(torch.bfloat16)
    half = R.gated_input(out, torch.zeros_like(out))
    assert torch.equal(half, (out.double() / 2).to(torch.bfloat16))
    assert torch.equal(R.gated_input(out, torch.full_like(out, 30.0)), out)
    assert float(R.gated_input(out, torch.full_like(out, -30.0)).abs().max()) < 1e-11 * float(out.abs().max())
    gate = (torch.randn(5, 96, generator=g) * 3).to(torch.bfloat16)
    y = R.gated_input(out, gate)
    exact = out.double() / (1 + torch.exp(-gate.double()))
    assert torch.all((y.double() - exact).abs() <= exact.abs() * 2.0 ** -7 + 1e-30)
    # the gate is the sigmoid's argument, not the product's other factor
    assert not torch.equal(y, R.gated_input(gate, out))


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_gated_rmsnorm_matches_transformers_module(wdtype):
    """core.py:390 applies transformers' Qwen3_5RMSNormGated to rows of head_v_dim (the module in the
    model dtype, trtllm_stack.py:198): the restatement equals the module itself, bit for bit."""
    Qwen3_5RMSNormGated = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5").Qwen3_5RMSNormGated
    g = gen(31)
    hd, heads = 128, 4
    x = (torch.randn(6, heads * hd, generator=g) * 2).to(torch.bfloat16)
    z = (torch.randn(6, heads * hd, generator=g) * 2).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hd, generator=g)).to(wdtype)
    mod = Qwen3_5RMSNormGated(hd, eps=1e-6).to(dtype=wdtype)
    with torch.no_grad():
        mod.weight.copy_(w)
        ref = mod(x.reshape(-1, hd), z.reshape(-1, hd)).reshape(x.shape)
    assert torch.equal(R.gated_rmsnorm(x, z, w, 1e-6, hd), ref)
    # known answers: z = 0 gates everything to 0; per-head (not per-row) normalization
    assert torch.equal(R.gated_rmsnorm(x, torch.zeros_like(z), w, 1e-6, hd), torch.zeros_like(x))
    scaled = x.clone()
    scaled[:, :hd] *= 4  # head 0 scaled by a power of two: its normalized values, and only its, stay put
    a, b = R.gated_rmsnorm(x, z, w, 1e-6, hd), R.gated_rmsnorm(scaled, z, w, 1e-6, hd)
    assert torch.allclose(a.float(), b.float(), rtol=2 ** -7, atol=1e-6)
    # heads of 2 hd (the same gain repeated) normalize over other groups: a wrong head split shows
    assert not torch.equal(R.gated_rmsnorm(x, z, w, 1e-6, hd), R.gated_rmsnorm(x, z, torch.cat([w, w]), 1e-6, 2 * hd))


def test_split_query_gate_takes_the_second_half_of_each_head():
    """core.py:231-232: q_proj rows viewed as [heads, 2 head_dim]; the gate is each head's second half."""
    heads, hd = 3, 8
    row = torch.arange(2 * heads * hd, dtype=torch.float32)
    query, gate = R.split_query_gate(row.reshape(1, -1).to(torch.bfloat16), hd)
    want = torch.cat([row[h * 2 * hd + hd:(h + 1) * 2 * hd] for h in range(heads)])
    assert torch.equal(gate.float().reshape(-1), want)
    assert torch.equal(query.float().reshape(-1), torch.cat([row[h * 2 * hd:h * 2 * hd + hd] for h in range(heads)]))


def test_outlier_generator_draw_order():
    g = gen(0)
    x = R.outlier_activations(g, 128, 1024)
    g2 = gen(0)
    base = torch.randn(128, 1024, generator=g2)
    idx = torch.randperm(1024, generator=g2)[:10]
    assert torch.equal(x[:, idx].float(), (base[:, idx] * 20).to(torch.bfloat16).float())
    big = (x.float().abs() > 10).float().mean(0)
    assert int((big > 0.3).sum()) == 10
