"""GPU: the benchmark configurations that the per-layer tests do not cover at their own workload.

- config 1: the Llama-3.2-1B FFN (H = 2048, I = 8192, g = 128) at one row, loaded from the reference's 4352-byte
  tiles, bf16 (the reference operator's type), against the float64 oracle;
- config 4: a random-init Llama-3-8B FFN stack (32 distinct layers, RMSNorm with eps 1e-5 and a residual add between
  them, attention omitted) decoding 128 tokens at one row: every layer of every step bit-equal to the separate
  rmsnorm -> forward -> residual_add2 path, x finite throughout with max|x| logged per layer, and steps 0 and 127
  checked layer by layer against the float64 oracle block (oracle/hm_oracle.c or_ffn_block_f64) with the same
  rounding points;
- RMSNorm where eps matters (|x| ~ 1e-3): eps sits inside the root (src/hipkernels/rmsnorm.cu:48)."""

import numpy as np
import pytest
import torch

from gpu_util import TORCH, assert_close, dev, dev_bits, host_bits, host_f64, make_x

pytestmark = pytest.mark.gpu


def test_config1_llama32_1b_decode_from_tiles(oracle, hm, device):
    rng = np.random.default_rng(1)
    h, inter, dtype = 2048, 8192, "bf16"
    ws = [oracle.random_weights(rng, h, inter, 128, dtype), oracle.random_weights(rng, h, inter, 128, dtype),
          oracle.random_weights(rng, inter, h, 128, dtype)]
    tiles = [dev(oracle.pack_tiles(*w), device) for w in ws]
    layer = hm.FfnLayer.from_tiles(*tiles, h, inter, dtype=torch.bfloat16)
    for m in (1, 1, 4):
        x64, x = make_x(oracle, rng, m, h, dtype, device)
        y = layer.forward(x)
        torch.cuda.synchronize()
        ref, _ = oracle.ffn(x64, *ws, 128, dtype)
        assert_close(oracle, host_f64(y), ref, dtype, f"config 1 Llama-3.2-1B FFN M={m}")
    # the same row through the restated reference CPU path (bf16, model-path SwiGLU) lands within its own tolerance
    x_bits = host_bits(x[0])
    y_cpu, _ = oracle.cpu_ffn_decode(x_bits, *[oracle.pack_tiles(*w) for w in ws], h, inter, threads=8)
    e = oracle.errors(oracle.bf16_bits_to_f32(y_cpu), ref[0])
    print(f"config 1 CPU baseline vs float64: {e}", flush=True)
    assert e["rel_l2"] < 1e-2


def _stack_layer(oracle, seed, hidden, inter, dtype):
    rng = np.random.default_rng(seed)
    return [oracle.random_weights(rng, hidden, inter, 128, dtype), oracle.random_weights(rng, hidden, inter, 128, dtype),
            oracle.random_weights(rng, inter, hidden, 128, dtype)]


def test_config4_llama3_8b_stack_128_steps(oracle, hm, device):
    hidden, inter, n_layers, steps, dtype, eps = 4096, 14336, 32, 128, "fp16", 1e-5
    check_steps = (0, steps - 1)
    layers, host_w, norm_bits, norm_w = [], [], [], []
    for li in range(n_layers):
        ws = _stack_layer(oracle, 4000 + li, hidden, inter, dtype)
        dw = [tuple(dev(t, device) if t.dtype == np.uint8 else dev_bits(t, dtype, device) for t in w) for w in ws]
        layers.append(hm.FfnLayer.from_logical(*dw, 128, dtype=TORCH[dtype]))
        del dw
        host_w.append(ws)
        nb = oracle.to_bits(np.random.default_rng(9000 + li).uniform(0.5, 1.5, hidden).astype(np.float32), dtype)
        norm_bits.append(nb)
        norm_w.append(dev_bits(nb, dtype, device))
    torch.cuda.synchronize()
    print(f"config 4: {n_layers} layers built", flush=True)
    mismatches = torch.zeros((), dtype=torch.int64, device=device)
    nonfinite = torch.zeros((), dtype=torch.int64, device=device)
    max_abs = torch.zeros(n_layers, dtype=torch.float32, device=device)
    saved = {s: [] for s in check_steps}  # layer inputs, then the final output
    normed = torch.empty((1, hidden), dtype=TORCH[dtype], device=device)
    for s in range(steps):
        _, x0 = make_x(oracle, np.random.default_rng(5000 + s), 1, hidden, dtype, device)  # a new token each step
        xa, xb = x0.clone(), x0.clone()
        for li in range(n_layers):
            if s in saved:
                saved[s].append(xa.clone())
            layers[li].block_forward(xa, norm_w[li], eps)  # two launches: norm in the gate_up GEMV, residual in the down
            hm.rmsnorm(normed, xb, norm_w[li], eps)  # the separate path
            y = layers[li].forward(normed)
            hm.residual_add2(xb, y)
            mismatches += (xa.view(torch.int16) != xb.view(torch.int16)).sum()
            nonfinite += (~torch.isfinite(xa)).sum()
            max_abs[li] = torch.maximum(max_abs[li], xa.float().abs().max())
        if s in saved:
            saved[s].append(xa.clone())
    torch.cuda.synchronize()
    print(f"config 4: {steps} steps done; max|x| per layer: {np.round(max_abs.cpu().numpy(), 1).tolist()}", flush=True)
    assert int(mismatches) == 0, f"{int(mismatches)} elements differ between block_forward and the separate ops"
    assert int(nonfinite) == 0
    # Steps 0 and 127 layer by layer against the float64 block, from the GPU's own input to each layer (so rounding
    # differences do not compound): the output x after the layer.
    worst = {"rel_l2": 0.0, "max_rel": 0.0}
    equal_bits = []
    for li in range(n_layers):
        for s in check_steps:
            xin = host_bits(saved[s][li][0])
            got = host_bits(saved[s][li + 1][0])
            out = oracle.ffn_block_f64(xin, norm_bits[li], eps, *host_w[li], 128, dtype, threads=16)
            e = oracle.errors(oracle.from_bits(got, dtype), oracle.from_bits(out["x_out"], dtype))
            worst = {k: max(worst[k], e[k]) for k in worst}
            equal_bits.append(float(np.mean(got == out["x_out"])))
            assert e["max_rel"] <= 1e-2 and e["rel_l2"] <= 1e-3, (li, s, e)
        host_w[li] = None  # free the host weights as we go
    print(f"config 4 vs float64 block (steps {check_steps}): worst {worst}, equal output bits {np.mean(equal_bits):.4f}", flush=True)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_rmsnorm_eps_matters_at_small_x(oracle, hm, device, dtype):
    # |x| ~ 1e-3: mean(x^2) ~ 1e-6 against eps = 1e-5, so the normalized values depend on where eps sits. The kernel
    # must match the oracle (eps inside the root, pinned by a closed form on the CPU), and the one-row block path
    # (the norm inside the gate_up GEMV) must give the same bits as the separate kernel.
    rng = np.random.default_rng(123)
    h, eps = 4096, 1e-5
    x64, x = make_x(oracle, rng, 3, h, dtype, device, scale=1e-3)
    w = torch.from_numpy(rng.uniform(0.5, 1.5, h).astype(np.float32)).to(device).to(TORCH[dtype])
    w64 = host_f64(w.view(1, -1))[0]
    out = torch.empty_like(x)
    hm.rmsnorm(out, x, w, eps)
    torch.cuda.synchronize()
    ref = oracle.rmsnorm(x64, w64, eps)
    assert_close(oracle, host_f64(out), ref, dtype, "rmsnorm |x|~1e-3")
    wrong = x64 / (np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True)) + eps) * w64  # eps outside the root
    assert oracle.errors(host_f64(out), wrong)["rel_l2"] > 0.5
    rng2 = np.random.default_rng(7)
    ws = [oracle.random_weights(rng2, h, 1024, 128, dtype), oracle.random_weights(rng2, h, 1024, 128, dtype),
          oracle.random_weights(rng2, 1024, h, 128, dtype)]
    layer = hm.FfnLayer.from_logical(*[tuple(dev(t, device) if t.dtype == np.uint8 else dev_bits(t, dtype, device) for t in wt) for wt in ws],
                                     128, dtype=TORCH[dtype])
    xa = x[:1].clone()
    layer.block_forward(xa, w, eps)
    xb = x[:1].clone()
    normed = torch.empty_like(xb)
    hm.rmsnorm(normed, xb, w, eps)
    hm.residual_add2(xb, layer.forward(normed))
    torch.cuda.synchronize()
    assert torch.equal(xa, xb)
