"""Graph and compile integration on the GPU.

* BackboneDecodeGraph (the reference's BackboneGraph decode step,
  models/cudagraph/backbone_graph.py:254-320) over a fused 3-layer Qwen3
  backbone with an fp32 head and CFG, captured once and replayed over
  positions with per-row padding, against the CPU float32 model running the
  same layers eagerly (bar 1e-2 on the CFG logits).
* torch.compile(fullgraph=True) over a module holding Int4Linear / Fp8Linear
  (the reference compiles its depth-decoder layers,
  models/cudagraph/depth_decoder_graph.py:164-192): the GEMV custom op traces
  without graph breaks and gives the eager result."""

from __future__ import annotations

import copy
import types

import numpy as np
import pytest
import torch
from torch import nn

from oracle import bz_oracle as O

from breeze_amd import fp8_linear as F8
from breeze_amd import int4_linear as I4
from breeze_amd.fused.graph import BackboneDecodeGraph
from breeze_amd.fused.install import install_fused_backbone, static_cache

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _model(layers=3, seed=7):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    cfg = Qwen3Config(hidden_size=512, intermediate_size=1024, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, num_hidden_layers=layers, rms_norm_eps=1e-6, max_position_embeddings=4096,
                      vocab_size=64)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    m = Qwen3Model(cfg).float().eval()
    with torch.no_grad():
        for p in m.parameters():
            (p.normal_(0, 0.03) if p.dim() == 2 else p.normal_(1, 0.1))
            p.copy_(p.to(torch.bfloat16).float())
    head = nn.Linear(512, 130, bias=False)
    with torch.no_grad():
        head.weight.normal_(0, 0.05)
    return cfg, m, head


def test_backbone_decode_graph_matches_cpu_model():
    cfg, ref, head = _model()
    gpu = copy.deepcopy(ref).to("cuda", torch.bfloat16)
    install_fused_backbone(types.SimpleNamespace(backbone_model=gpu), batch_size=2, max_seq_len=48)
    B, S, scale = 2, 48, 1.7
    g = BackboneDecodeGraph(gpu, copy.deepcopy(head).cuda(), batch_size=B, max_seq_len=S, guidance_scale=scale)
    g.pad_lens.copy_(torch.tensor([0, 2]))
    gen = torch.Generator().manual_seed(3)
    xs = [torch.randn(B, 1, 512, generator=gen).to(torch.bfloat16).float() for _ in range(10)]
    g.set_step(xs[0].cuda(), 0)
    g.capture(num_warmup=1)
    g.reset()

    c_ref = static_cache(cfg, S, B)
    mask = torch.full((B, 1, 1, S), torch.finfo(torch.float32).min)
    for t, x in enumerate(xs):
        out = g.step(x.to("cuda", torch.bfloat16), t).float().cpu().numpy()
        pid = torch.full((B, 1), t)
        kv = torch.arange(S)
        valid = (kv >= torch.tensor([0, 2]).unsqueeze(1)) & (kv <= t)
        mask.fill_(torch.finfo(torch.float32).min)
        mask[:, 0, 0, :] = mask[:, 0, 0, :].masked_fill(valid, 0.0)
        with torch.no_grad():
            h = x
            pe = ref.rotary_emb(h, pid)
            for layer in ref.layers:
                h = layer(h, attention_mask=mask, position_ids=pid, past_key_values=c_ref, use_cache=True,
                          position_embeddings=pe)
                h = h[0] if isinstance(h, tuple) else h
            h = ref.norm(h)[:, -1, :]
        logits = O.linear_f32_ref(h.numpy(), head.weight.detach().numpy())
        cfg_ref = logits[1:2] + scale * (logits[0:1] - logits[1:2])
        if t >= 2:  # row 1 attends to nothing before position 2
            assert O.rel_err(out, cfg_ref) <= TOL, t


def test_compile_fullgraph_with_quantized_linears():
    torch.manual_seed(0)

    class _MLP(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = nn.Linear(512, 1024, bias=False)
            self.up_proj = nn.Linear(512, 1024, bias=False)
            self.down_proj = nn.Linear(1024, 512, bias=False)

        def forward(self, x):
            return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))

    for quant in (I4.quantize_module_int4, F8.quantize_module_fp8):
        m = _MLP().to("cuda", torch.bfloat16)
        quant(m, min_bytes=0)
        x = torch.randn(2, 1, 512, device="cuda").to(torch.bfloat16)
        eager = m(x)
        compiled = torch.compile(m, fullgraph=True, backend="aot_eager")
        got = compiled(x)
        assert torch.equal(got, eager)
        np.testing.assert_array_equal(compiled(x * 2).float().cpu().numpy(), m(x * 2).float().cpu().numpy())


@pytest.mark.parametrize("quant", ["int4", "fp8"])
def test_inductor_compile_then_graph_capture(quant):
    """The reference's depth-decoder flow (models/cudagraph/
    depth_decoder_graph.py:164-192; test_fp8_linear.py:38-63): a module
    holding Int4Linear / Fp8Linear compiled with the default backend
    (inductor, mode="default", fullgraph=True), then captured in a HIP graph
    and replayed.  The GEMV custom op stays one opaque launch; inductor
    generates the glue (SiLU-mul, residual add) itself, in fp32 where eager
    torch rounds the SiLU to bf16 first, so the compiled module is held to
    the 1e-2 bar against the uncompiled one, and every graph replay to the
    compiled module's eager result bit for bit."""
    torch.manual_seed(1)

    class _Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = nn.Linear(512, 1024, bias=False)
            self.up_proj = nn.Linear(512, 1024, bias=False)
            self.down_proj = nn.Linear(1024, 512, bias=False)

        def forward(self, x):
            return x + self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))

    m = _Block().to("cuda", torch.bfloat16)
    (I4.quantize_module_int4 if quant == "int4" else F8.quantize_module_fp8)(m, min_bytes=0)
    x = torch.randn(2, 1, 512, device="cuda").to(torch.bfloat16)
    eager = m(x)
    compiled = torch.compile(m, mode="default", fullgraph=True)
    want = compiled(x)
    assert O.rel_err(want.float().cpu().numpy(), eager.float().cpu().numpy()) <= TOL
    static_x = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # warm-up calls outside the capture
            compiled(static_x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        out = compiled(static_x)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        _ = (x.float() * 3).sum().item()  # eager work between the replays
    static_x.copy_(x * 2)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, compiled(x * 2))
