"""GPU-resident fused decode-GEMM behind torch.nn.Linear (GPU only).

ResidentLinear keeps a layer's .xksv blocks in HBM and computes x @ W.T with
the fused kernels; install_resident_linear swaps it into a model the way the
reference installs its fused GEMV (python/runtime.py:248-287).  Checks:
  * the layer against an fp64 product of the same bf16 operands: rel-L2
    <= 1e-5 with fp32 output, <= 2e-3 after rounding the output to bf16;
  * the GPU-decode load (decode_weight) bit-exact against the weight;
  * a tiny Llama (transformers, random init) with every linear layer but
    lm_head resident: logits within atol = rtol = 0.03 of the same model with
    plain layers, for a 3-token prefill and one cached decode step -- the
    reference's bound for its fused path (tests/test_stream.py:54-62).
    Attention runs in fp32 (eager), so no bf16 batched products are involved.
"""
from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

import xksv_hip
import xksv_torch

pytestmark = pytest.mark.gpu


def _rel_l2(got, want):
    got = np.asarray(got.detach() if isinstance(got, torch.Tensor) else got, np.float64)
    want = np.asarray(want.detach() if isinstance(want, torch.Tensor) else want, np.float64)
    return np.linalg.norm(got - want) / np.linalg.norm(want)


@pytest.mark.parametrize("out_f,in_f,codec", [(512, 4096, 2), (256, 1024, 1), (1024, 512, 2), (40, 4096, 2)])
@pytest.mark.parametrize("tokens", [1, 3, 8, 17])
@torch.no_grad()
def test_resident_linear_matches_fp64(hip, out_f, in_f, codec, tokens):
    torch.manual_seed(out_f + in_f + tokens)
    lin = torch.nn.Linear(in_f, out_f, bias=tokens % 2 == 1, device="cuda", dtype=torch.bfloat16)
    torch.nn.init.normal_(lin.weight, std=0.02)
    rl = xksv_torch.ResidentLinear.from_linear(hip, lin, codec)
    x = torch.randn(tokens, in_f, device="cuda", dtype=torch.float32)
    xb = x.to(torch.bfloat16)
    want = xb.double() @ lin.weight.double().T
    if lin.bias is not None:
        want += lin.bias.double()
    y32 = rl(xb.float())  # fp32 in -> fp32 out (the product of the bf16-rounded x)
    assert y32.dtype == torch.float32 and y32.shape == (tokens, out_f)
    assert _rel_l2(y32.cpu(), want.cpu()) <= 1e-5
    y16 = rl(xb.reshape(1, tokens, in_f))
    assert y16.dtype == torch.bfloat16 and y16.shape == (1, tokens, out_f)
    assert _rel_l2(y16.float().cpu().reshape(tokens, out_f), want.cpu()) <= 2e-3


@torch.no_grad()
def test_resident_linear_decode_weight_bit_exact(hip):
    torch.manual_seed(3)
    lin = torch.nn.Linear(4096, 96, bias=False, device="cuda", dtype=torch.bfloat16)
    torch.nn.init.normal_(lin.weight, std=0.02)
    for codec in (1, 2):
        rl = xksv_torch.ResidentLinear.from_linear(hip, lin, codec)
        assert rl.archive.numel() < lin.weight.numel() * 2  # stored compressed
        assert torch.equal(rl.decode_weight().view(torch.int16), lin.weight.view(torch.int16))


@torch.no_grad()
def test_resident_linear_reports_corrupt_blocks(hip):
    torch.manual_seed(4)
    lin = torch.nn.Linear(4096, 64, bias=False, device="cuda", dtype=torch.bfloat16)
    torch.nn.init.normal_(lin.weight, std=0.02)
    rl = xksv_torch.ResidentLinear.from_linear(hip, lin, 2)
    first = int(rl._decode_table[0]["offset"])
    rl.archive[first] ^= 1  # XKSP2 magic of block 0
    rl(torch.randn(1, 4096, device="cuda"))  # recorded on the device, no host sync
    with pytest.raises(xksv_hip.XksvError):
        rl.check_errors()
    rl.check = True
    with pytest.raises(xksv_hip.XksvError):
        rl(torch.randn(2, 4096, device="cuda", dtype=torch.bfloat16))


@pytest.mark.parametrize("tokens", [1, 5])
@torch.no_grad()
def test_resident_linear_fp32_activations(hip, tokens):
    """fp32 activations take the fp32-X path (the reference's fused GEMV numerics,
    python/runtime.py:267): rel-L2 <= 1e-5 against fp64 with the unrounded fp32 x."""
    torch.manual_seed(40 + tokens)
    lin = torch.nn.Linear(4096, 384, bias=True, device="cuda", dtype=torch.bfloat16)
    torch.nn.init.normal_(lin.weight, std=0.02)
    rl = xksv_torch.ResidentLinear.from_linear(hip, lin, 2)
    x = torch.randn(tokens, 4096, device="cuda", dtype=torch.float32)
    want = x.double() @ lin.weight.double().T + lin.bias.double()
    y = rl(x)
    assert y.dtype == torch.float32
    assert _rel_l2(y.cpu(), want.cpu()) <= 1e-5
    rl.check_errors()


@torch.no_grad()
def test_resident_linear_forward_under_graph_capture(hip):
    """forward issues no host synchronisation: it captures into a HIP graph, and
    every replay (with eager work and synchronisations between replays) equals
    the eager result bit for bit, for the fp32 and the bf16 (MFMA) paths."""
    torch.manual_seed(77)
    lin = torch.nn.Linear(4096, 256, bias=False, device="cuda", dtype=torch.bfloat16)
    torch.nn.init.normal_(lin.weight, std=0.02)
    rl = xksv_torch.ResidentLinear.from_linear(hip, lin, 2)
    xs = {torch.float32: torch.randn(3, 4096, device="cuda"),
          torch.bfloat16: torch.randn(8, 4096, device="cuda").to(torch.bfloat16)}
    for dt, x in xs.items():
        eager = rl(x).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            rl(x)  # warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = rl(x)
        for i in range(3):
            x.add_(0)  # eager work between replays
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager), (dt, i)
    rl.check_errors()


def test_tiny_llama_logits_with_resident_layers(hip):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                                   attn_implementation="eager")
    torch.manual_seed(712)
    base = transformers.LlamaForCausalLM(cfg).eval()
    for m in base.modules():  # bf16-valued linear weights, fp32 everywhere else
        if isinstance(m, torch.nn.Linear):
            m.weight.data = m.weight.data.to(torch.bfloat16).float()
    base = base.to("cuda")
    fused = copy.deepcopy(base)
    for name, m in fused.named_modules():
        if isinstance(m, torch.nn.Linear) and not name.endswith("lm_head"):
            m.weight.data = m.weight.data.to(torch.bfloat16)
    assert xksv_torch.install_resident_linear(fused, hip) == 14
    assert isinstance(fused.model.layers[1].mlp.down_proj, xksv_torch.ResidentLinear)
    ids = torch.tensor([[1, 2, 1]], device="cuda")
    with torch.inference_mode():
        a = fused(input_ids=ids, use_cache=True)
        b = base(input_ids=ids, use_cache=True)
        assert torch.allclose(a.logits, b.logits, atol=0.03, rtol=0.03)
        nxt = b.logits[:, -1, :].argmax(-1, keepdim=True)
        a2 = fused(input_ids=nxt, past_key_values=a.past_key_values, use_cache=True)
        b2 = base(input_ids=nxt, past_key_values=b.past_key_values, use_cache=True)
        assert torch.allclose(a2.logits, b2.logits, atol=0.03, rtol=0.03)
