"""End-to-end generation on the GPU through ``dLLM.generate`` for the three model families
(random-initialised shape presets): every step kind runs (full, sparse refresh, sparse
Q-pruned), every answer position is unmasked, and generation is deterministic."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _run(model, prompts, sp, threshold=0.99):
    from dyllm_amd import dLLM

    eng = dLLM(model, threshold=threshold)
    out = eng.generate(prompts, sp)
    torch.cuda.synchronize()
    return eng, out


@pytest.mark.parametrize("model", ["tiny-llada", "tiny-dream", "tiny-llada-moe"])
def test_generate_all_step_kinds(dev, model):
    from dyllm_amd import SamplingParams

    print(f"[engine] {model}", flush=True)
    sp = SamplingParams(max_new_tokens=64, steps=16, num_full_steps=2, block_size=16, temperature=0.0)
    prompts = [[3, 14, 15, 92, 65], [2, 71, 82, 81, 82, 84, 59], [1] * 12]
    eng, out = _run(model, prompts, sp)
    mask = eng.config.mask_id
    assert len(out) == 3
    for o, p in zip(out, prompts):
        ids = o["token_ids"]
        assert ids[: len(p)] == p
        assert len(ids) == len(p) + 64
        # a random-initialised model may itself emit the mask id (the reference does not suppress
        # it either), so only most answer positions are guaranteed to hold real tokens
        assert ids[len(p):].count(mask) < 16 or eng.config.eos in ids[len(p):]
    st = eng.execution_stats
    assert st["full_forwards"] == 2 and st["sparse_forwards"] >= 6     # refresh and Q-pruned steps ran
    _, out2 = _run(model, prompts, sp)
    assert [o["token_ids"] for o in out] == [o["token_ids"] for o in out2]


def test_generate_confidence_threshold_and_batches(dev):
    """Sequences admitted at different times (a new one joins while others are sparse) and the
    confidence-threshold unmasking rule."""
    from dyllm_amd import SamplingParams, dLLM

    eng = dLLM("tiny-llada", threshold=0.99, max_num_seqs=2)
    sp = SamplingParams(max_new_tokens=32, steps=8, num_full_steps=1, block_size=8, temperature=0.0,
                        confidence_threshold=0.0)      # every candidate qualifies: a block per step
    out = eng.generate([[5, 6, 7], [8, 9], [10, 11, 12, 13]], sp)
    for o in out:
        assert eng.config.mask_id not in o["token_ids"]
    assert eng.execution_stats["full_forwards"] >= 2


def test_host_staging_single_transfer(dev):
    """The step metadata travels in one pinned transfer; every field comes back with its dtype and
    values, also when the pinned buffer is reused by the next step while the device block of the
    previous one is still referenced."""
    from dyllm_amd.engine.model_runner import _HostStaging

    st = _HostStaging(torch.device(dev))
    rng = torch.Generator().manual_seed(3)
    kept = []
    for step in range(3):
        fields = {"a": (torch.randint(-2**40, 2**40, (1000 + step,), generator=rng), torch.long),
                  "b": (torch.randint(-2**30, 2**30, (7,), generator=rng).to(torch.int32), torch.int32),
                  "e": (torch.zeros(0, dtype=torch.long), torch.long),
                  "c": (torch.randn(33, generator=rng), torch.float32)}
        for name, (t, dt) in fields.items():
            st.add(name, t.tolist(), dt)
        out = st.flush()
        kept.append((fields, out))
    torch.cuda.synchronize()
    for fields, out in kept:
        for name, (t, dt) in fields.items():
            assert out[name].dtype == dt and out[name].device.type == "cuda"
            assert torch.equal(out[name].cpu(), t.to(dt)), name


def test_generate_config4_long_context(dev):
    """Config 4 through dLLM.generate: the LLaDA-8B shape (32 layers, random-init bf16), batch 2,
    2048 prompt + 6144 response tokens (an 8192-row context, past the checkpoint's 4096 positions,
    so the RoPE tables are raised to 8192), tau = 0.995, a full-attention refresh every 8 steps."""
    from dyllm_amd import SamplingParams, dLLM

    print("[engine] config4 long context", flush=True)
    eng = dLLM("llada-8b", threshold=0.995, max_model_len=8192, max_position_embeddings=8192, refresh_period=8)
    assert eng.config.max_model_len == 8192
    rot = eng.model_runner.model.model.layers[0].self_attn.rotary
    assert rot.cos.shape[0] == 8192
    g = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, 126000, (2048,), generator=g).tolist() for _ in range(2)]
    steps = 24
    sp = SamplingParams(max_new_tokens=6144, steps=steps, num_full_steps=1, block_size=6144, temperature=0.0)
    out = eng.generate(prompts, sp)
    torch.cuda.synchronize()
    st = eng.execution_stats
    assert st["full_forwards"] == 1 and st["full_forwards"] + st["sparse_forwards"] == steps
    # processed steps 9-15 and 17-23 are Q-pruned; 2-8, 16 and 24 query every row
    assert eng.model_runner.num_q_pruned_forwards == 14
    for o, p in zip(out, prompts):
        assert o["token_ids"][:2048] == p and len(o["token_ids"]) == 8192
        assert o["token_ids"][2048:].count(eng.config.mask_id) < 6144 // 8


@pytest.mark.parametrize("model", ["tiny-llada", "tiny-dream", "tiny-llada-moe"])
def test_device_bookkeeping_same_tokens(dev, model):
    """Sparse steps of a running batch built on the device (dyllm_unmask_step: commit, salient
    lists, input ids, sampler candidates) generate the same tokens as host-built steps, with
    fixed-count and confidence-threshold unmasking and a batch that changes mid-run."""
    from dyllm_amd import SamplingParams, dLLM

    print(f"[engine] device bookkeeping {model}", flush=True)
    outs, dev_steps = [], []
    for on in (False, True):
        eng = dLLM(model, threshold=0.99, max_num_seqs=3)
        eng.model_runner.device_bookkeeping = on
        sps = [SamplingParams(max_new_tokens=64, steps=16, num_full_steps=2, block_size=16, temperature=0.0),
               SamplingParams(max_new_tokens=48, steps=12, num_full_steps=3, block_size=8, temperature=0.0,
                              confidence_threshold=0.05),
               SamplingParams(max_new_tokens=64, steps=16, num_full_steps=2, block_size=16, temperature=0.0)]
        prompts = [[3, 14, 15, 92, 65], [2, 71, 82, 81, 82, 84, 59], [1] * 12, [9, 9, 8]]
        out = eng.generate(prompts, sps + [sps[0]])
        torch.cuda.synchronize()
        outs.append([o["token_ids"] for o in out])
        dev_steps.append(eng.model_runner.device_steps)
    assert dev_steps[0] == 0 and dev_steps[1] > 10
    assert outs[0] == outs[1]


def test_device_bookkeeping_same_tokens_sampled(dev):
    """With a temperature (Dream samples categorically), device-built steps draw from the random
    generator exactly as host-built ones do: the sampler runs on the valid candidates only, in
    the host path's order, so both give the same tokens from the same seed."""
    from dyllm_amd import SamplingParams, dLLM

    outs, dev_steps = [], []
    for on in (False, True):
        eng = dLLM("tiny-dream", threshold=0.99, max_num_seqs=3)
        eng.model_runner.device_bookkeeping = on
        sp = SamplingParams(max_new_tokens=48, steps=12, num_full_steps=2, block_size=16, temperature=0.8)
        torch.manual_seed(1234)
        out = eng.generate([[3, 14, 15, 92, 65], [2, 71, 82, 81], [1] * 9], sp)
        torch.cuda.synchronize()
        outs.append([o["token_ids"] for o in out])
        dev_steps.append(eng.model_runner.device_steps)
    assert dev_steps[0] == 0 and dev_steps[1] > 5
    assert outs[0] == outs[1]
