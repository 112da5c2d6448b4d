"""The reference's forward call sequence, compiled and graph-captured the way its model runner runs it.

miniagentserve/engine/model_runner.py:98 compiles the model with ``torch.compile(dynamic=True)`` and
:101-119 captures the compiled forward in CUDA graphs on a side stream after three warm-up calls.
Inside, the layer ops mutate *views*: RoPE rotates the q / k column views of the qkv GEMM output in
place (miniagentserve/models/devstral2/devstral2.py:158-166), the append reads views of the same
buffer (:170-173), decode and context attention write the ``[:d]`` and ``[d:]`` slices of one output
(:181-213), and the embedding gather (:282) follows the runner's placeholder fill
(model_runner.py:149-154). ``MiniModel`` below is that forward with two layers at small sizes and
with the GEMMs replaced by opaque elementwise stand-ins (below). Layer 0 uses the reference's
separate RoPE and append calls and its torch llama-4 query scale; layer 1 the fused RoPE + KV +
q-scale op.

The compiled, graph-replayed step must reproduce the eager step bit for bit: the final hidden
states, the residual stream, both KV caches and the resolved token ids. Run as a script
(``python tests/test_gpu_compiled_step.py``), the module replays the captured step a few times, for
a kernel trace of what one compiled step launches.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F
from torch import nn
from torch.library import custom_op

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


# GEMM stand-ins. Like the reference's FP8Linear (devstral2.py:100-115), each is an opaque op that
# returns a freshly allocated output, so the compiled graph holds qkv, the o_proj output and gate_up
# as realized buffers whose column views RoPE and the KV append mutate and read in place. Their
# values are elementwise, computed in eager torch inside the op, so eager and compiled runs agree.
@custom_op("mas_test::gemm_from_codes", mutates_args=())
def gemm_from_codes(x: torch.Tensor, base: torch.Tensor) -> torch.Tensor:
    """bf16(f32(base) + first fp8 code of each row of x, read as a byte): [rows, base width]."""
    return (base.float() + x.view(torch.uint8)[:, :1].float()).to(torch.bfloat16)


@gemm_from_codes.register_fake
def _(x, base):
    return base.new_empty((x.shape[0], base.shape[1]))


@custom_op("mas_test::gemm_scaled", mutates_args=())
def gemm_scaled(x: torch.Tensor, base: torch.Tensor, factor: float) -> torch.Tensor:
    """bf16(f32(x) * factor + f32(base)) with fp8 x read as bytes; x is [rows, base width]."""
    xf = x.view(torch.uint8).float() if x.dtype == FP8 else x.float()
    return (xf * factor + base.float()).to(torch.bfloat16)


@gemm_scaled.register_fake
def _(x, base, factor):
    return base.new_empty((x.shape[0], base.shape[1]))

# Small Devstral-shaped sizes: hidden = q_heads * head_dim so the o_proj stand-in is elementwise.
HIDDEN, INTER, HQ, HK, D, VOCAB, LAYERS = 512, 512, 4, 2, 128, 1000, 2
PAGES, PAGE_SIZE, WIDTH = 64, 16, 8          # the reference engine's default block size (serving_engine.py:24)
BETA, ORIG_MAX = 0.1, 64                      # llama-4 query scale: 1 + beta * log1p(floor(pos / 64))
EPS = 1e-5


class MiniModel(nn.Module):
    """Devstral2Model.forward (devstral2.py:267-308) with the decoder layer (:237-253) and attention
    (:155-214) inlined, at two layers; GEMM outputs are elementwise functions of their inputs."""

    def __init__(self, mas, device, seed: int = 0):
        super().__init__()
        self.mas = mas
        g = torch.Generator(device=device).manual_seed(seed)

        def randn(*shape, scale=1.0, shift=0.0):
            return (shift + scale * torch.randn(*shape, generator=g, device=device)).to(torch.bfloat16)

        self.embed = randn(VOCAB, HIDDEN)
        self.w_in = [randn(HIDDEN, scale=0.1, shift=1.0) for _ in range(LAYERS)]
        self.w_post = [randn(HIDDEN, scale=0.1, shift=1.0) for _ in range(LAYERS)]
        self.w_final = randn(HIDDEN, scale=0.1, shift=1.0)
        self.qkv_base = [randn(1, (HQ + 2 * HK) * D) for _ in range(LAYERS)]
        self.o_base = [randn(1, HIDDEN) for _ in range(LAYERS)]
        self.gu_base = [randn(1, 2 * INTER) for _ in range(LAYERS)]
        self.act_scale = torch.tensor(0.05, device=device)
        self.cos_sin = mas.rope.cos_sin_cache(WIDTH * PAGE_SIZE, D, 1e6).to(device)
        self.workspace = torch.zeros(8 << 20, dtype=torch.uint8, device=device)
        self.scaling = D ** -0.5

    def forward(self, input_ids, last_tokens, *, k_cache, v_cache, positions, batch_indices, seq_lens,
                cu_seqlens_q, block_tables, error_flags):
        mas = self.mas
        num_tokens, batch, num_prefills = input_ids.shape[0], seq_lens.shape[0], cu_seqlens_q.shape[0] - 1
        d = batch - num_prefills
        hidden = mas.embedding.embedding(input_ids, self.embed, last_tokens=last_tokens, error_flags=error_flags)
        kv_indptr = torch.arange(batch + 1, dtype=torch.int32, device=input_ids.device) * block_tables.shape[1]
        kv_last_page_len = (seq_lens - 1) % k_cache.shape[2] + 1
        residual = torch.zeros_like(hidden)
        for layer in range(LAYERS):
            kc, vc = k_cache[layer], v_cache[layer]
            x = torch.empty(hidden.shape, dtype=FP8, device=hidden.device)
            mas.fused_add_rmsnorm_quant(x, hidden, residual, self.w_in[layer], self.act_scale, EPS)
            qkv = gemm_from_codes(x, self.qkv_base[layer])                               # qkv_proj
            q, k, v = qkv.split([HQ * D, HK * D, HK * D], dim=-1)
            v = v.unflatten(-1, (-1, D))
            if layer == 0:
                mas.apply_rope_with_cos_sin_cache_inplace(positions, q, k, D, self.cos_sin, is_neox=True,
                                                          error_flags=error_flags)
                q = q.unflatten(-1, (-1, D))
                k = k.unflatten(-1, (-1, D))
                mas.append_paged_kv_cache(k, v, batch_indices, positions, (kc, vc), block_tables.flatten(),
                                          kv_indptr, kv_last_page_len, kv_layout="NHD", error_flags=error_flags)
                attn_scale = 1 + BETA * torch.log1p(torch.floor(positions.float() / ORIG_MAX))
                q = q * attn_scale[:, None, None].to(q.dtype)
            else:
                mas.apply_rope_and_append_paged_kv_cache(positions, q, k, v, D, self.cos_sin, True, batch_indices,
                                                         (kc, vc), block_tables.flatten(), kv_indptr,
                                                         kv_last_page_len, "NHD", llama_4_scaling_beta=BETA,
                                                         original_max_position_embeddings=ORIG_MAX,
                                                         error_flags=error_flags)
                q = q.unflatten(-1, (-1, D))
            attn_output = torch.empty(q.shape, dtype=q.dtype, device=q.device)
            if d:
                mas.attention.trtllm_batch_decode_with_kv_cache(
                    query=q[:d], kv_cache=(kc, vc), workspace_buffer=self.workspace, block_tables=block_tables[:d],
                    seq_lens=seq_lens[:d], max_seq_len=k_cache.shape[1] * k_cache.shape[2],
                    bmm1_scale=self.scaling, bmm2_scale=1.0, out=attn_output[:d], kv_layout="NHD",
                    error_flags=error_flags)
            if num_prefills:
                mas.attention.trtllm_batch_context_with_kv_cache(
                    query=q[d:], kv_cache=(kc, vc), workspace_buffer=self.workspace, block_tables=block_tables[d:],
                    seq_lens=seq_lens[d:], max_q_len=num_tokens - d, max_kv_len=block_tables.shape[1] * k_cache.shape[2],
                    bmm1_scale=self.scaling, bmm2_scale=1.0, batch_size=num_prefills, cum_seq_lens_q=cu_seqlens_q,
                    cum_seq_lens_kv=F.pad(seq_lens[d:].cumsum(0, dtype=torch.int32), (1, 0)), out=attn_output[d:],
                    kv_layout="NHD", error_flags=error_flags)
            hidden = gemm_scaled(attn_output.flatten(1), self.o_base[layer], 0.5)          # o_proj
            mas.fused_add_rmsnorm_quant(x, hidden, residual, self.w_post[layer], self.act_scale, EPS)
            gate_up = gemm_from_codes(x, self.gu_base[layer])                             # gate_up_proj
            y = mas.activation.silu_and_mul_quant(gate_up, self.act_scale)
            hidden = gemm_scaled(y, self.o_base[layer], 0.25)                             # down_proj
        mas.fused_add_rmsnorm(hidden, residual, self.w_final, EPS)
        return hidden, residual


def make_step_inputs(device, seed: int = 1):
    """One mixed step as ModelRunner.prepare lays it out (model_runner.py:176-225): 3 decode rows
    (one token each, ids are placeholders -1 - r for the previous step's samples), then 2 prompt rows
    (chunked prefill: 20 new tokens after 13 cached, and a fresh 27-token prompt); distinct pages."""
    g = torch.Generator().manual_seed(seed)
    decode_lens = [37, 101, 5]
    prompts = [(13, 20), (0, 27)]                                 # (cached, new) per prompt row
    batch = len(decode_lens) + len(prompts)
    tables = torch.randperm(PAGES, generator=g)[: batch * WIDTH].reshape(batch, WIDTH).to(torch.int32)
    ids, pos, idx = [], [], []
    for r, n in enumerate(decode_lens):
        ids.append(-1 - r)
        pos.append(n - 1)
        idx.append(r)
    cu = [0]
    for j, (cached, new) in enumerate(prompts):
        row = len(decode_lens) + j
        ids += torch.randint(0, VOCAB, (new,), generator=g).tolist()
        pos += list(range(cached, cached + new))
        idx += [row] * new
        cu.append(cu[-1] + new)
    seq_lens = decode_lens + [c + n for c, n in prompts]
    kv = (LAYERS, PAGES, PAGE_SIZE, HK, D)
    dg = torch.Generator(device=device).manual_seed(seed)
    return {
        "input_ids": torch.tensor(ids, dtype=torch.int64, device=device),
        "last_tokens": torch.randint(0, VOCAB, (len(decode_lens),), generator=g).to(torch.int32).to(device),
        "positions": torch.tensor(pos, dtype=torch.int32, device=device),
        "batch_indices": torch.tensor(idx, dtype=torch.int32, device=device),
        "seq_lens": torch.tensor(seq_lens, dtype=torch.int32, device=device),
        "cu_seqlens_q": torch.tensor(cu, dtype=torch.int32, device=device),
        "block_tables": tables.to(device),
        # cached positions hold earlier tokens' keys and values
        "k_cache": torch.randn(kv, generator=dg, device=device).to(torch.bfloat16),
        "v_cache": torch.randn(kv, generator=dg, device=device).to(torch.bfloat16),
        "error_flags": torch.zeros(1, dtype=torch.int32, device=device),
    }


def _run(model, inputs):
    kw = {k: v for k, v in inputs.items() if k not in ("input_ids", "last_tokens")}
    return model(inputs["input_ids"], inputs["last_tokens"], **kw)


class _Runner:
    """Holds static inputs, a pristine copy to reset them from, and the compiled, captured step."""

    def __init__(self, mas, device):
        self.model = MiniModel(mas, device)
        self.pristine = make_step_inputs(device)
        self.static = {k: v.clone() for k, v in self.pristine.items()}
        self.compiled = torch.compile(self.model, dynamic=True, fullgraph=True)

    def reset(self):
        for k, v in self.static.items():
            v.copy_(self.pristine[k])

    def eager(self):
        self.reset()
        out = _run(self.model, self.static)
        torch.cuda.synchronize()
        return self.snapshot(out)

    def snapshot(self, out):
        s = self.static
        return [out[0].clone(), out[1].clone(), s["k_cache"].clone(), s["v_cache"].clone(), s["input_ids"].clone(),
                s["error_flags"].clone()]

    def capture(self):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):                     # as model_runner.py:108-111
                self.reset()
                _run(self.compiled, self.static)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.reset()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.graph_out = _run(self.compiled, self.static)
        torch.cuda.synchronize()

    def replay(self):
        self.reset()
        torch.cuda.synchronize()
        self.graph.replay()
        torch.cuda.synchronize()
        return self.snapshot(self.graph_out)


def test_compiled_graph_step_matches_eager(mas, dev):
    runner = _Runner(mas, dev)
    want = runner.eager()
    assert int(want[5]) == 0, "eager step reported index errors"
    assert (want[4] >= 0).all(), "placeholders left unresolved"
    runner.capture()
    names = ["hidden", "residual", "k_cache", "v_cache", "input_ids", "error_flags"]
    for replay in range(3):                       # eager work and syncs between replays
        got = runner.replay()
        for name, a, b in zip(names, got, want):
            assert torch.equal(a, b), f"replay {replay}: {name} differs from eager"
        again = runner.eager()
        for name, a, b in zip(names, again, want):
            assert torch.equal(a, b), f"eager after replay {replay}: {name} differs"


def test_compiled_ops_report_error_bits(mas, dev):
    """error_flags travel through the compiled custom ops: a position past the cos/sin table sets the
    POSITION bit (2) and a page id past the cache sets the PAGE bit (8), as in eager mode."""
    g = torch.Generator(device=dev).manual_seed(4)
    table = mas.rope.cos_sin_cache(32, D, 1e6).to(dev)
    kc = torch.zeros(4, PAGE_SIZE, HK, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)

    def f(qkv, positions, batch_indices, kv_indices, kv_indptr, flags):
        q, k, v = qkv.split([HQ * D, HK * D, HK * D], dim=-1)
        mas.apply_rope_with_cos_sin_cache_inplace(positions, q, k, D, table, True, error_flags=flags)
        mas.append_paged_kv_cache(k.unflatten(-1, (-1, D)), v.unflatten(-1, (-1, D)), batch_indices, positions,
                                  (kc, vc), kv_indices, kv_indptr, None, "NHD", error_flags=flags)
        return qkv + 0

    qkv = torch.randn(3, (HQ + 2 * HK) * D, generator=g, device=dev).to(torch.bfloat16)
    positions = torch.tensor([1, 40, 3], dtype=torch.int32, device=dev)      # 40 is past the 32-row table
    batch_indices = torch.zeros(3, dtype=torch.int32, device=dev)
    kv_indices = torch.tensor([0, 1, 9], dtype=torch.int32, device=dev)      # position 40 -> entry 2: page 9,
                                                                              # past the 4-page cache
    kv_indptr = torch.tensor([0, 3], dtype=torch.int32, device=dev)
    results = []
    for fn in (f, torch.compile(f, dynamic=True, fullgraph=True)):
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        kc.zero_()
        vc.zero_()
        out = fn(qkv.clone(), positions, batch_indices, kv_indices, kv_indptr, flags)
        torch.cuda.synchronize()
        results.append((int(flags), out, kc.clone()))
    assert results[0][0] == results[1][0] == (2 | 8)
    assert torch.equal(results[0][1], results[1][1]) and torch.equal(results[0][2], results[1][2])


if __name__ == "__main__":
    # Kernel-trace driver: capture the compiled step, then replay it 5 times.
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    device = torch.device("cuda:0")
    r = _Runner(pkg, device)
    want_ = r.eager()
    r.capture()
    torch.cuda.synchronize()
    print("captured; replaying", flush=True)
    for _ in range(5):
        got_ = r.replay()
        assert all(torch.equal(a, b) for a, b in zip(got_, want_))
    print("compiled step: 5 graph replays bit-equal to eager", flush=True)
