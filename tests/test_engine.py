"""CPU checks of the host-side engine around the hot path: configuration parsing, the
scheduler's full -> sparse progression and retirement rules, the sampler against a per-sequence
brute force, the sparse-step index construction, the generate loop (with a stand-in model
runner), and safetensors loading with LLaDA's checkpoint names."""
import json
import os

import pytest
import torch

from dyllm_amd.config import Config, ModelConfig, PRESETS
from dyllm_amd.engine.model_runner import ModelRunner
from dyllm_amd.engine.scheduler import Scheduler
from dyllm_amd.engine.sequence import Sequence, SequenceStatus
from dyllm_amd.model_executor.layers.sampler import DreamSampler, LLaDASampler
from dyllm_amd.sampling_params import SamplingParams
from dyllm_amd.utils.context import get_context, reset_context, set_context
from dyllm_amd.utils.metadata import reset_metadata

MASK, EOS = 511, 510


def test_config_from_llada_json(tmp_path):
    d = dict(model_type="llada", d_model=256, n_heads=2, n_kv_heads=2, n_layers=3, mlp_hidden_size=512,
             vocab_size=500, embedding_size=512, max_sequence_length=1024, rope_theta=500000.0, rms_norm_eps=1e-5,
             mask_token_id=MASK, eos_token_id=EOS, include_bias=False, weight_tying=False)
    (tmp_path / "config.json").write_text(json.dumps(d))
    cfg = Config(str(tmp_path), max_model_len=4096)
    hf = cfg.hf_config
    assert (hf.hidden_size, hf.num_attention_heads, hf.num_hidden_layers, hf.intermediate_size) == (256, 2, 3, 512)
    assert hf.vocab_size == 512 and hf.head_dim == 128 and not hf.is_moe
    assert cfg.mask_id == MASK and cfg.eos == EOS and cfg.max_model_len == 1024
    assert cfg.model_dir == str(tmp_path)


def test_config_presets_and_errors():
    c = Config("dream-7b")
    assert c.hf_config.model_type == "Dream" and c.hf_config.num_key_value_heads == 4 and c.hf_config.qkv_bias
    assert Config("llada-moe-7b").hf_config.is_moe
    assert Config("llada-8b").hf_config.intermediate_size == 12288
    with pytest.raises(ValueError, match="one GPU"):
        Config("llada-8b", tensor_parallel_size=2)
    with pytest.raises(ValueError, match="preset"):
        Config("/nonexistent/model")


def _seq(prompt_len, new, **kw):
    sp = SamplingParams(max_new_tokens=new, mask_id=MASK, **kw)
    return Sequence(list(range(1, prompt_len + 1)) + [MASK] * new, sp)


def test_scheduler_full_then_sparse():
    cfg = Config("tiny-llada")
    sch = Scheduler(cfg)
    seqs = [_seq(4, 8, steps=4, num_full_steps=2, block_size=8) for _ in range(3)]
    for s in seqs:
        sch.add(s)
    kinds = []
    for _ in range(4):
        batch, full = sch.schedule()
        assert [s.seq_id for s in batch] == [s.seq_id for s in seqs]
        kinds.append(full)
    assert kinds == [True, True, False, False]
    assert all(s.status == SequenceStatus.SPARSE for s in seqs)
    assert all(s.processed_steps == 4 for s in seqs)


def test_scheduler_retires_on_eos_and_on_steps():
    cfg = Config("tiny-llada")
    sch = Scheduler(cfg)
    a = _seq(2, 4, steps=2, num_full_steps=1, block_size=4)
    b = _seq(2, 4, steps=2, num_full_steps=1, block_size=4)
    sch.add(a)
    sch.add(b)
    batch, full = sch.schedule()
    assert full
    # a: EOS at its first answer position with nothing masked before it -> finished
    # b: two ordinary tokens, one step of two left
    pos = torch.tensor([[2, 0], [2, 3]])
    tok = torch.tensor([[EOS, -1], [7, 8]])
    cnt = torch.tensor([1, 2], dtype=torch.int32)
    fin = sch.postprocess(batch, pos, tok, cnt)
    assert fin == [a.seq_id] and a.is_finished and not b.is_finished
    assert b.token_ids[2:4] == [7, 8] and b.num_completion_tokens == 2
    batch, full = sch.schedule()
    assert not full and batch == [b]
    fin = sch.postprocess(batch, torch.tensor([[4, 5]]), torch.tensor([[9, 9]]), torch.tensor([2], dtype=torch.int32))
    assert fin == [b.seq_id] and sch.is_finished()


def _brute_sample(logits, cu_q, cands, offsets, n_transfer, thr, block):
    """Per sequence: softmax over the vocabulary, confidence = max prob, stable order by
    descending confidence, keep the first n_transfer or any with confidence >= thr."""
    out = []
    for b, rel in enumerate(cands):
        items = []
        for r in rel[:block]:
            p = torch.softmax(logits[cu_q[b] + r], dim=-1)
            items.append((float(p.max()), int(p.argmax()), r + offsets[b]))
        order = sorted(range(len(items)), key=lambda i: -items[i][0])
        keep = [items[i] for j, i in enumerate(order) if j < n_transfer[b] or items[i][0] >= thr[b]]
        out.append([(t, p) for _, t, p in keep])
    return out


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_sampler_matches_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    V, block = 64, 8
    cu_q = [0, 12, 20, 33]
    logits = torch.randn(cu_q[-1], V, generator=g) * 3
    cands = [[1, 4, 5, 9, 11], [0, 2, 3, 4, 5, 6, 7, 1, 3], []]      # seq 1 has more than one block
    offsets = [0, 100, 7]
    n_transfer = [2, 3, 1]
    thr = [float("inf"), 0.3, float("inf")]
    set_context(False, cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32))
    rel = torch.tensor([r for c in cands for r in c], dtype=torch.long)
    cu = torch.tensor([0, 5, 14, 14], dtype=torch.int32)
    pos, tok, cnt = LLaDASampler("confidence")(logits, get_context(), (rel, torch.tensor(offsets), cu),
                                                num_transfer=torch.tensor(n_transfer), block_size=block,
                                                confidence_thresholds=torch.tensor(thr))
    reset_context()
    want = _brute_sample(logits, cu_q, cands, offsets, n_transfer, thr, block)
    for b in range(3):
        n = int(cnt[b])
        got = list(zip(tok[b, :n].tolist(), pos[b, :n].tolist()))
        assert got == want[b], (b, got, want[b])
        assert (tok[b, n:] == -1).all()


def test_dream_sampler_shift_and_entropy():
    logits = torch.tensor([[0.0, 5.0, 0.0], [9.0, 0.0, 0.0], [0.0, 0.0, 1.0]])
    s = DreamSampler("entropy")
    shifted = s.adjust_logits(logits)
    assert torch.equal(shifted[1], logits[0]) and torch.equal(shifted[0], logits[0])
    p = torch.softmax(shifted, -1)
    sc = s.compute_scores(p, p.max(-1).values)
    assert sc.argmax().item() == 2          # row 2 now holds the most peaked logits: highest -entropy


def _runner_cpu(cfg):
    return ModelRunner(cfg, model=torch.nn.Identity(), device="cpu")


def test_prepare_sparse_indices():
    reset_metadata()
    cfg = Config("tiny-llada")
    r = _runner_cpu(cfg)
    a, b = _seq(3, 8), _seq(5, 8)
    a.last_token_pos, b.last_token_pos = [4, 1, 9], [5, 12]     # position 1 is in a's prompt
    for s in (a, b):
        s.processed_steps = 8                                       # refresh step (multiple of 4)
    r.prepare_sparse([a, b])(r.staging.flush())
    ctx = get_context()
    assert ctx.cu_seqlens_q_cpu == [0, 11, 24] and ctx.idx_salient_row_k is None
    assert ctx.idx_salient_row.tolist() == [4, 9, 11 + 5, 11 + 12]
    assert ctx.cu_salientlens.tolist() == [0, 2, 4] and ctx.max_salientlen == 2
    for s in (a, b):
        s.processed_steps = 6                                       # Q-pruned step
    ids, pos = r.prepare_sparse([a, b])(r.staging.flush())
    assert pos.tolist() == list(range(3, 11)) + list(range(5, 13)) and ids.dtype == torch.long
    ctx = get_context()
    assert ctx.cu_seqlens_q_cpu == [0, 8, 16] and ctx.cu_promptlens.tolist() == [0, 3, 8]
    assert ctx.idx_salient_row.tolist() == [1, 6, 8 + 0, 8 + 7]
    assert ctx.idx_salient_row_k.tolist() == [4, 9, 11 + 5, 11 + 12]
    assert ctx.cu_seqlens_k.dtype == torch.int32 and ctx.idx_salient_row.dtype == torch.long
    reset_context()


class _FakeRunner:
    """Stands in for the GPU model runner: unmasks the first num_transfer masked positions of
    the current block with token (position % 5) + 1, never EOS."""

    def __init__(self):
        self.num_full_forwards = self.num_sparse_forwards = 0

    def call(self, method, seqs, is_full, finished):
        if is_full:
            self.num_full_forwards += 1
        else:
            self.num_sparse_forwards += 1
        W = max(s.block_size for s in seqs)
        pos = torch.zeros(len(seqs), W, dtype=torch.long)
        tok = torch.full((len(seqs), W), -1, dtype=torch.long)
        cnt = torch.zeros(len(seqs), dtype=torch.int32)
        for b, s in enumerate(seqs):
            lim = min(len(s), s.block_size * (s.block_idx + 1) + s.num_prompt_tokens)
            m = [i for i in range(lim) if s.token_ids[i] == MASK][: s.num_transfer_tokens]
            for j, p in enumerate(m):
                pos[b, j], tok[b, j] = p, p % 5 + 1
            cnt[b] = len(m)
        return pos, tok, cnt


def test_generate_loop_with_stand_in_runner():
    from dyllm_amd import SamplingParams as SP, dLLM

    eng = dLLM("tiny-llada", threshold=0.99, model_runner=_FakeRunner())
    sp = SP(max_new_tokens=16, steps=8, num_full_steps=3, block_size=8, temperature=0.0)
    out = eng.generate([[5, 6, 7], [1, 2, 3, 4, 5]], sp)
    assert len(out) == 2
    for o, plen in zip(out, (3, 5)):
        ids = o["token_ids"]
        assert len(ids) == plen + 16 and MASK not in ids
        assert ids[plen:] == [p % 5 + 1 for p in range(plen, plen + 16)]
        assert o["text"] == ""                          # no tokenizer files for a preset
    assert eng.execution_stats == {"full_forwards": 3, "sparse_forwards": 5}
    with pytest.raises(ValueError, match="token-id"):
        eng.generate(["hello"], sp)


def test_weight_loader_llada_names(tmp_path):
    from safetensors.torch import save_file

    from dyllm_amd.model_executor.models import model_class
    from dyllm_amd.utils.weight_loader import load_model

    hf = PRESETS["tiny-llada"]
    src = model_class(hf)(hf, 0.99, device="cpu", seed=1)
    dst = model_class(hf)(hf, 0.99, device="cpu", seed=2)
    I, kv = hf.intermediate_size, hf.num_key_value_heads * hf.head_dim
    t = {"model.transformer.wte.weight": src.model.embed_tokens.data,
         "model.transformer.ln_f.weight": src.model.norm.weight.data,
         "model.transformer.ff_out.weight": src.lm_head.data}
    for i, layer in enumerate(src.model.layers):
        p = f"model.transformer.blocks.{i}."
        at, mlp = layer.self_attn, layer.mlp
        t[p + "q_proj.weight"] = at.q_proj.data
        t[p + "k_proj.weight"] = at.kv_proj.data[:kv]
        t[p + "v_proj.weight"] = at.kv_proj.data[kv:]
        t[p + "attn_out.weight"] = at.o_proj.data
        t[p + "ff_proj.weight"] = mlp.gate_up_proj.data[:I]
        t[p + "up_proj.weight"] = mlp.gate_up_proj.data[I:]
        t[p + "ff_out.weight"] = mlp.down_proj.data
        t[p + "attn_norm.weight"] = layer.input_layernorm.weight.data * 2
        t[p + "ff_norm.weight"] = layer.post_attention_layernorm.weight.data * 3
    save_file({k: v.contiguous() for k, v in t.items()}, str(tmp_path / "model.safetensors"))
    load_model(dst, str(tmp_path))
    sd_src, sd_dst = dict(src.named_parameters()), dict(dst.named_parameters())
    for k, v in sd_src.items():
        want = v.data
        if k.endswith("input_layernorm.weight"):
            want = want * 2
        if k.endswith("post_attention_layernorm.weight"):
            want = want * 3
        assert torch.equal(sd_dst[k].data, want), k
    del t["model.transformer.blocks.0.up_proj.weight"]
    save_file({k: v.contiguous() for k, v in t.items()}, str(tmp_path / "model.safetensors"))
    with pytest.raises(RuntimeError, match="unset"):
        load_model(model_class(hf)(hf, 0.99, device="cpu"), str(tmp_path))


def test_weight_loader_moe_experts():
    from dyllm_amd.model_executor.models import model_class
    from dyllm_amd.utils.weight_loader import load_weights

    hf = PRESETS["tiny-llada-moe"]
    src = model_class(hf)(hf, 0.99, device="cpu", seed=3)
    dst = model_class(hf)(hf, 0.99, device="cpu", seed=4)
    I = hf.expert_intermediate_size
    ws = []
    for n, p in src.named_parameters():
        if n.endswith("mlp.gate_up_proj"):
            for e in range(hf.num_experts):
                ws.append((n.replace("gate_up_proj", f"experts.{e}.gate_proj.weight"), p.data[e, :I]))
                ws.append((n.replace("gate_up_proj", f"experts.{e}.up_proj.weight"), p.data[e, I:]))
        elif n.endswith("mlp.down_proj"):
            for e in range(hf.num_experts):
                ws.append((n.replace("down_proj", f"experts.{e}.down_proj.weight"), p.data[e]))
        elif n.endswith("kv_proj"):
            h = p.shape[0] // 2
            ws.append((n.replace("kv_proj", "k_proj.weight"), p.data[:h]))
            ws.append((n.replace("kv_proj", "v_proj.weight"), p.data[h:]))
        elif n.endswith(".weight"):
            ws.append((n, p.data))
        else:
            ws.append((n + ".weight", p.data))
    load_weights(dst, ws)
    for (n, a), (_, b) in zip(src.named_parameters(), dst.named_parameters()):
        assert torch.equal(a.data, b.data), n


def test_config_refresh_period_and_long_context():
    """Config 4: refresh every 8 steps and an 8192-row context on the LLaDA-8B shape, whose
    checkpoint caps positions at 4096 (config.py:51-58 clips max_model_len to it)."""
    from dyllm_amd.engine.model_runner import q_pruned_step

    assert Config("llada-8b", max_model_len=8192).max_model_len == 4096   # the reference's clip
    c = Config("llada-8b", max_model_len=8192, max_position_embeddings=8192, refresh_period=8)
    assert c.max_model_len == 8192 and c.hf_config.max_position_embeddings == 8192
    assert PRESETS["llada-8b"].max_position_embeddings == 4096            # the preset is not mutated
    with pytest.raises(ValueError, match="refresh_period"):
        Config("llada-8b", refresh_period=0)

    class _S:
        processed_steps = 0

    def kinds(period):
        out = []
        for n in range(1, 25):
            _S.processed_steps = n
            out.append("q" if q_pruned_step(_S, period) else "r")
        return "".join(out)

    # period 4 is the reference's cadence (model_runner.py:211)
    assert kinds(4) == "rrrr" + "qqqr" * 5
    assert kinds(8) == "rrrrrrrr" + "qqqqqqqr" * 2
