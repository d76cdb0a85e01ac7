"""Builds the per-step batch and context, runs the model and the sampler
(dyllm/engine/model_runner.py:20-549, the mask-based model path on one GPU).

Step kinds (model_runner.py:140-298):

* full      -- every row of every sequence is queried; the layers run dense attention and the
               FFN over all rows and rewrite their caches;
* sparse    -- the first layer's salient rows are the positions the previous step unmasked;
               each layer's attention decides the next layer's salient rows. After
               `refresh_period` (4) processed steps a sparse step queries only the response rows
               (Q-pruned), except every `refresh_period`-th step, which queries all rows (refresh).

A batch is Q-pruned only when all its sequences are (the reference decides per sequence but
then drops the K-space index list as soon as one sequence refreshes, model_runner.py:213-220,
which leaves a mixed batch inconsistent); batches of sequences admitted together, the case the
scheduler produces, behave identically.
"""
from __future__ import annotations

from typing import List, Optional

import numpy as np
import torch

from ..config import Config
from ..model_executor.layers.sampler import DenseCandidates, DreamSampler, LLaDASampler, RowLogits
from ..utils.context import get_context, reset_context, set_context
from ..utils.metadata import get_metadata
from .sequence import Sequence


def build_model(config: Config, device="cuda"):
    from ..model_executor.models import model_class

    hf = config.hf_config
    cls = model_class(hf)
    model = cls(hf, config.threshold, device=device, seed=config.seed)
    wdir = config.model_dir
    if wdir is not None:
        from ..utils.weight_loader import has_safetensors, load_model

        if has_safetensors(wdir):
            load_model(model, wdir)
    return model


_NP_DTYPE = {torch.int32: np.int32, torch.long: np.int64, torch.float32: np.float32}


class _HostStaging:
    """One host-to-device transfer per step for all of its index / offset metadata (the reference
    issues one small copy per tensor, model_runner.py:140-298). Fields are packed 16-byte aligned
    into a reusable pinned buffer and copied with one non-blocking copy into a fresh device block;
    each field comes back as a typed view of that block. The pinned buffer is rewritten only after
    the previous copy out of it has completed."""

    def __init__(self, device: torch.device):
        self.device = device
        self.fields = []
        self.pinned = None
        self.copied = None   # event recorded after the last copy out of `pinned`

    def add(self, name: str, data, dtype) -> None:
        self.fields.append((name, np.ascontiguousarray(np.asarray(data, dtype=_NP_DTYPE[dtype])), dtype))

    def flush(self) -> dict:
        offs, n = [], 0
        for _, arr, _ in self.fields:
            offs.append(n)
            n += (arr.nbytes + 15) // 16 * 16
        fields, self.fields = self.fields, []
        if self.device.type != "cuda":
            return {name: torch.from_numpy(arr.copy()).to(self.device) for name, arr, _ in fields}
        if self.copied is not None:
            self.copied.synchronize()
        if self.pinned is None or self.pinned.numel() < n:
            cap = max(n, 2 * self.pinned.numel() if self.pinned is not None else 1 << 16)
            self.pinned = torch.empty(cap, dtype=torch.uint8, pin_memory=True)
        host = self.pinned.numpy()
        for (_, arr, _), o in zip(fields, offs):
            host[o:o + arr.nbytes] = arr.view(np.uint8).reshape(-1)
        dev = torch.empty(max(n, 16), dtype=torch.uint8, device=self.device)
        dev[:n].copy_(self.pinned[:n], non_blocking=True)
        self.copied = torch.cuda.Event()
        self.copied.record()
        return {name: dev[o:o + arr.nbytes].view(dt) for (name, arr, dt), o in zip(fields, offs)}


class _DeviceBatch:
    """Device-resident state of one running batch between its sparse steps: the token rows (packed
    by cu_seqlens_k), the generated-token counters, the per-sequence layout and sampling knobs, and
    the previous sampler output. A step of the same batch is then built on the device by one
    ``dyllm_unmask_step`` launch (commit + salient lists + input ids + sampler candidates) instead
    of host lists; the host keeps only the sizes it launches with (from its mirrors). Built from
    the host mirrors before a host-built step's output is committed; dropped when the batch
    changes."""

    def __init__(self, runner: "ModelRunner", seqs: List[Sequence]):
        dev = runner.device
        cfg = runner.config
        self.ids = [s.seq_id for s in seqs]
        B = len(seqs)
        lens = [len(s) for s in seqs]
        cu_k = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        astart = [s.answer_start for s in seqs]
        prompt = [s.num_prompt_tokens for s in seqs]
        i32 = lambda x: torch.as_tensor(np.asarray(x), dtype=torch.int32, device=dev)
        self.lens, self.cu_k_cpu = lens, cu_k.tolist()
        self.tok = torch.from_numpy(np.concatenate([s.token_arr for s in seqs])).to(dev)
        self.cu_k, self.prompt, self.astart = i32(cu_k), i32(prompt), i32(astart)
        self.astart_cpu = astart
        self.cu_p = i32(np.concatenate([[0], np.cumsum(prompt)]))
        self.block = i32([s.block_size for s in seqs])
        self.generated = i32([s.num_completion_tokens for s in seqs])
        self.lens_t = i32(lens)
        self.seq_ids = torch.tensor(self.ids, dtype=torch.long, device=dev)
        self.W = max(s.block_size if s.block_size is not None else s.max_new_tokens for s in seqs)
        W = self.W
        # the two step layouts: Q-pruned (answer rows) and refresh (every row)
        cu_q = np.concatenate([[0], np.cumsum([L - a for L, a in zip(lens, astart)])]).astype(np.int64)
        pos_p = np.concatenate([np.arange(a, L, dtype=np.int64) for L, a in zip(lens, astart)])
        pos_r = np.concatenate([np.arange(L, dtype=np.int64) for L in lens])
        self.layout = {
            True: (cu_q.tolist(), i32(cu_q), torch.from_numpy(pos_p).to(dev), i32(astart)),
            False: (self.cu_k_cpu, self.cu_k, torch.from_numpy(pos_r).to(dev), i32([0] * B)),
        }
        # per-sequence sampling knobs ([B]; None when no sequence sets one), as prepare_sample
        temps = [s.temperature if (s.temperature is not None and s.temperature > 1e-6) else 1.0 for s in seqs]
        has_t = any(s.temperature is not None and s.temperature > 1e-6 for s in seqs)
        f32 = lambda x: torch.tensor(x, dtype=torch.float32, device=dev)
        self.temps = f32(temps) if has_t else None
        self.top_ks = i32([s.top_k if s.top_k is not None else 1 << 30 for s in seqs]) \
            if any(s.top_k is not None for s in seqs) else None
        self.top_ps = f32([s.top_p if s.top_p is not None else 1.0 for s in seqs]) \
            if any(s.top_p is not None for s in seqs) else None
        self.thrs = f32([s.confidence_threshold if s.confidence_threshold is not None else float("inf")
                         for s in seqs]) if any(s.confidence_threshold is not None for s in seqs) else None
        self.transfers = i32([1 if s.confidence_threshold is not None else s.num_transfer_tokens for s in seqs])
        # outputs of the device build (capacities: every sampled slot, every queried row)
        cap = max(B * W, 1)
        self.idx_q = torch.empty(cap, dtype=torch.long, device=dev)
        self.idx_q32 = torch.empty(cap, dtype=torch.int32, device=dev)
        self.idx_k = torch.empty(cap, dtype=torch.long, device=dev)
        self.idx_k32 = torch.empty(cap, dtype=torch.int32, device=dev)
        self.idx_upd = torch.empty(cap, dtype=torch.int32, device=dev)
        self.pos_k = torch.empty(cap, dtype=torch.long, device=dev)
        self.cu_s = torch.empty(B + 1, dtype=torch.int32, device=dev)
        self.input_ids = torch.empty(max(int(cu_q[-1]), 1), dtype=torch.long, device=dev)
        self.cand_rel = torch.empty(B, W, dtype=torch.long, device=dev)
        self.cand_n = torch.empty(B, dtype=torch.int32, device=dev)
        # previous sampled set: the host mirrors' last written positions (each sequence's salient
        # rows when this step samples nothing for it, as the host path)
        lp = torch.zeros(B, W, dtype=torch.long)
        lt = torch.zeros(B, W, dtype=torch.long)
        lc = torch.zeros(B, dtype=torch.int32)
        for b, s in enumerate(seqs):
            n = min(len(s.last_token_pos), W)
            lp[b, :n] = torch.tensor(s.last_token_pos[:n], dtype=torch.long)
            lt[b, :n] = torch.tensor(s.last_tokens[:n], dtype=torch.long)
            lc[b] = n
        self.last = (lp.to(dev), lt.to(dev), lc.to(dev))

    def matches(self, seqs: List[Sequence]) -> bool:
        return [s.seq_id for s in seqs] == self.ids

    def record(self, pos, tok, cnt):
        """Keep this step's sampler output; a sequence that sampled nothing keeps its previous set."""
        lp, lt, lc = self.last
        got = (cnt > 0)
        self.last = (torch.where(got.unsqueeze(1), pos.long(), lp), torch.where(got.unsqueeze(1), tok.long(), lt),
                     torch.where(got, cnt.to(torch.int32), lc))


def q_pruned_step(seq: Sequence, period: int = 4) -> bool:
    """Sparse step that queries only the response rows (model_runner.py:211, period 4 there):
    after `period` processed steps, all but every `period`-th step."""
    return seq.processed_steps > period and seq.processed_steps % period != 0


class ModelRunner:

    def __init__(self, config: Config, rank: int = 0, event=None, model=None, device="cuda"):
        self.config = config
        self.rank = rank
        self.device = torch.device(device)
        self.num_full_forwards = 0
        self.num_sparse_forwards = 0
        self.num_q_pruned_forwards = 0     # sparse steps that queried only the response rows
        hf = config.hf_config
        self.model = model if model is not None else build_model(config, device)
        self.sampler = DreamSampler("entropy") if hf.model_type == "Dream" else LLaDASampler("confidence")
        self.staging = _HostStaging(self.device)
        self._dev_batch: Optional[_DeviceBatch] = None   # state of the running sparse batch
        self.device_bookkeeping = True                   # build repeated sparse steps on the device
        self.device_steps = 0                            # sparse steps built on the device

    # -- batch preparation -------------------------------------------------------------
    def prepare_full(self, seqs: List[Sequence]):
        md = get_metadata()
        cu, lens, ids = [0], [], []
        for seq in seqs:
            L = len(seq)
            cu.append(cu[-1] + L)
            lens.append(L)
            ids.append(seq.seq_id)
        input_ids = np.concatenate([seq.token_arr for seq in seqs])
        positions = np.concatenate([np.arange(L, dtype=np.int64) for L in lens])
        i32, i64 = torch.int32, torch.long
        st = self.staging
        st.add("cu", cu, i32)
        st.add("ids", ids, i64)
        st.add("lens", lens, i32)
        st.add("input_ids", input_ids, i64)
        st.add("positions", positions, i64)

        def finish(d):
            md.running_seqs = ids
            md.running_seqs_tensor = d["ids"]
            set_context(True, cu_seqlens_q=d["cu"], cu_seqlens_q_cpu=cu, cu_seqlens_k=d["cu"], cu_seqlens_k_cpu=cu,
                        max_seqlen_q=max(lens), max_seqlen_k=max(lens), context_lens=d["lens"],
                        context_lens_cpu=lens, total_seqlen=cu[-1], total_seqlen_k=cu[-1])
            return d["input_ids"], d["positions"]

        return finish

    def prepare_sparse(self, seqs: List[Sequence]):
        md = get_metadata()
        pruned = all(q_pruned_step(s, self.config.refresh_period) for s in seqs)
        input_ids, positions, positions_k = [], [], []
        idx_q, idx_k, idx_upd = [], [], []
        cu_q, cu_k, cu_p, cu_s, lens, ids = [0], [0], [0], [0], [], []
        for seq in seqs:
            L = len(seq)
            start = seq.answer_start
            kept = [p for p in seq.last_token_pos if p >= start]
            if pruned:
                input_ids.append(seq.token_arr[start:])
                positions.append(np.arange(start, L, dtype=np.int64))
                idx_q.extend(p - seq.num_prompt_tokens + cu_q[-1] for p in kept)
                idx_k.extend(p + cu_k[-1] for p in kept)
                lq = L - start
            else:
                input_ids.append(seq.token_arr)
                positions.append(np.arange(L, dtype=np.int64))
                idx_q.extend(p + cu_q[-1] for p in kept)
                lq = L
            positions_k.extend(kept)
            idx_upd.extend(p + cu_k[-1] for p in kept)
            cu_p.append(cu_p[-1] + seq.num_prompt_tokens)
            cu_s.append(cu_s[-1] + len(kept))
            cu_q.append(cu_q[-1] + lq)
            cu_k.append(cu_k[-1] + L)
            lens.append(L)
            ids.append(seq.seq_id)
        i32, i64 = torch.int32, torch.long
        st = self.staging
        for name, data, dt in (("cu_s", cu_s, i32), ("ids", ids, i64), ("idx_q", idx_q, i64), ("cu_q", cu_q, i32),
                               ("cu_k", cu_k, i32), ("cu_p", cu_p, i32), ("idx_upd", idx_upd, i32),
                               ("idx_k", idx_k, i64), ("lens", lens, i32), ("positions_k", positions_k, i64),
                               ("input_ids", np.concatenate(input_ids), i64),
                               ("positions", np.concatenate(positions), i64)):
            st.add(name, data, dt)

        def finish(d):
            md.running_seqs = ids
            md.running_seqs_tensor = d["ids"]
            set_context(False, cu_seqlens_q=d["cu_q"], cu_seqlens_q_cpu=cu_q, cu_seqlens_k=d["cu_k"],
                        cu_seqlens_k_cpu=cu_k, cu_promptlens=d["cu_p"], cu_updatedlens=d["cu_s"],
                        cu_salientlens=d["cu_s"], max_seqlen_q=max(cu_q[i + 1] - cu_q[i] for i in range(len(seqs))),
                        max_seqlen_k=max(lens), idx_updated_row=d["idx_upd"], idx_salient_row=d["idx_q"],
                        idx_salient_row_k=d["idx_k"] if pruned else None,
                        max_salientlen=max(cu_s[i + 1] - cu_s[i] for i in range(len(seqs))),
                        context_lens=d["lens"], context_lens_cpu=lens, total_seqlen_k=cu_k[-1],
                        total_seqlen=cu_q[-1], positions_k=d["positions_k"])
            return d["input_ids"], d["positions"]

        return finish

    def prepare_sample(self, seqs: List[Sequence], pruned: bool):
        """Candidate rows of the current block and the per-sequence sampling knobs
        (model_runner.py:300-372); staged with the step's other metadata."""
        mask = self.config.mask_id
        rels, counts, temps, transfers, top_ps, top_ks, thrs, offsets = [], [], [], [], [], [], [], []
        has_t = has_p = has_k = has_thr = False
        for seq in seqs:
            limit = min(len(seq), seq.block_size * (seq.block_idx + 1) + seq.num_prompt_tokens)
            mpos = np.flatnonzero(seq.token_arr[:limit] == mask)
            off = seq.answer_start if pruned else 0
            if pruned:
                mpos = mpos[mpos >= off] - off
            n = len(mpos)
            rels.append(mpos)
            offsets.append(off)
            counts.append(n)
            t_on = seq.temperature is not None and seq.temperature > 1e-6
            has_t |= t_on
            # sequences without a temperature are left unscaled in a batch that has one
            temps.append(np.full(n, seq.temperature if t_on else 1.0))
            transfers.append(1 if seq.confidence_threshold is not None else seq.num_transfer_tokens)
            top_ps.append(np.full(n, seq.top_p if seq.top_p is not None else 1.0))
            top_ks.append(np.full(n, seq.top_k if seq.top_k is not None else 1 << 30))
            thrs.append(seq.confidence_threshold if seq.confidence_threshold is not None else float("inf"))
            has_p |= seq.top_p is not None
            has_k |= seq.top_k is not None
            has_thr |= seq.confidence_threshold is not None
        block = max(s.block_size if s.block_size is not None else s.max_new_tokens for s in seqs)
        cu = [0]
        for c in counts:
            cu.append(cu[-1] + c)
        f32, i32, i64 = torch.float32, torch.int32, torch.long
        st = self.staging
        if has_t:
            st.add("s_temps", np.concatenate(temps), f32)
        if has_k:
            st.add("s_top_ks", np.concatenate(top_ks), i32)
        if has_p:
            st.add("s_top_ps", np.concatenate(top_ps), f32)
        if has_thr:
            st.add("s_thrs", thrs, f32)
        st.add("s_rels", np.concatenate(rels), i64)
        st.add("s_offsets", offsets, i64)
        st.add("s_cu", cu, i32)
        st.add("s_transfers", transfers, i32)

        def finish(d):
            params = (d.get("s_temps"), d.get("s_top_ks"), d.get("s_top_ps"), block, d.get("s_thrs"))
            return params, (d["s_rels"], d["s_offsets"], d["s_cu"]), d["s_transfers"]

        return finish

    # -- execution ------------------------------------------------------------------------
    @torch.inference_mode()
    def run_model(self, input_ids, positions, is_full: bool):
        """Hidden states of every queried row; the LM head runs later on the sampler's candidate
        rows only (RowLogits)."""
        return RowLogits(self.model(input_ids, positions), self.model.compute_logits)

    def _host_candidates(self, seqs: List[Sequence], pruned: bool, width: int) -> int:
        """Candidates of the step from the host mirrors (the masked positions of the current block,
        at most `width` per sequence): the count unmask_step_kernel writes to cand_n, summed."""
        mask = self.config.mask_id
        total = 0
        for seq in seqs:
            limit = min(len(seq), seq.block_size * (seq.block_idx + 1) + seq.num_prompt_tokens)
            off = seq.answer_start if pruned else 0
            total += min(width, int(np.count_nonzero(seq.token_arr[off:limit] == mask)) if limit > off else 0)
        return total

    def _run_device_step(self, db: _DeviceBatch, seqs: List[Sequence], pruned: bool):
        """A sparse step of the same batch as the previous one, built on the device."""
        from .. import _lib
        md = get_metadata()
        B = len(seqs)
        cu_q_cpu, cu_q, positions, offsets = db.layout[pruned]
        lp, lt, lc = db.last
        _lib.call("dyllm_unmask_step", db.tok.data_ptr(), db.cu_k.data_ptr(), B, lp.data_ptr(), lt.data_ptr(),
                  lc.data_ptr(), lp.shape[1], db.generated.data_ptr(), db.prompt.data_ptr(), db.astart.data_ptr(),
                  db.block.data_ptr(), int(self.config.mask_id), int(pruned), cu_q.data_ptr(), db.idx_q.data_ptr(),
                  db.idx_q32.data_ptr(), db.idx_k.data_ptr(), db.idx_k32.data_ptr(), db.idx_upd.data_ptr(),
                  db.pos_k.data_ptr(), db.cu_s.data_ptr(), db.input_ids.data_ptr() if pruned else None,
                  db.cand_rel.data_ptr(), db.cand_n.data_ptr(), db.W, torch.cuda.current_stream().cuda_stream)
        # host-side sizes from the mirrors (updated by the scheduler from the same sampled set)
        kept = [sum(1 for p in s.last_token_pos if p >= a) for s, a in zip(seqs, db.astart_cpu)]
        n = sum(kept)
        md.running_seqs = db.ids
        md.running_seqs_tensor = db.seq_ids
        idx_k = db.idx_k[:n]
        set_context(False, cu_seqlens_q=cu_q, cu_seqlens_q_cpu=cu_q_cpu, cu_seqlens_k=db.cu_k,
                    cu_seqlens_k_cpu=db.cu_k_cpu, cu_promptlens=db.cu_p, cu_updatedlens=db.cu_s,
                    cu_salientlens=db.cu_s, max_seqlen_q=max(cu_q_cpu[i + 1] - cu_q_cpu[i] for i in range(B)),
                    max_seqlen_k=max(db.lens), idx_updated_row=db.idx_upd[:n], idx_salient_row=db.idx_q[:n],
                    idx_salient_row_i32=db.idx_q32[:n], idx_salient_row_k=idx_k if pruned else None,
                    max_salientlen=max(kept), context_lens=db.lens_t, context_lens_cpu=db.lens,
                    total_seqlen_k=db.cu_k_cpu[-1], total_seqlen=cu_q_cpu[-1], positions_k=db.pos_k[:n])
        input_ids = db.input_ids[:cu_q_cpu[-1]] if pruned else db.tok
        logits = self.run_model(input_ids, positions, False)
        with torch.inference_mode():
            pos, tok, cnt = self.sampler(input_logits=logits, ctx=get_context(),
                                         input_indices=DenseCandidates(db.cand_rel, db.cand_n, offsets,
                                                                       self._host_candidates(seqs, pruned, db.W)),
                                         temperatures=db.temps, num_transfer=db.transfers, top_k=db.top_ks,
                                         top_p=db.top_ps, block_size=db.W, confidence_thresholds=db.thrs)
        db.record(pos, tok, cnt)
        reset_context()
        self.device_steps += 1
        return pos, tok, cnt

    def run(self, seqs: List[Sequence], is_full: bool, finished_seqs: Optional[List[int]] = None):
        if is_full:
            self.num_full_forwards += 1
        else:
            self.num_sparse_forwards += 1
        get_metadata().finished_seqs = list(finished_seqs or [])
        db = self._dev_batch
        if not is_full and self.device.type == "cuda" and db is not None and db.matches(seqs):
            pruned = all(q_pruned_step(s, self.config.refresh_period) for s in seqs)
            self.num_q_pruned_forwards += int(pruned)
            return self._run_device_step(db, seqs, pruned)
        # host-built step; a sparse batch keeps a device state for its following steps
        self._dev_batch = db = None
        if not is_full and self.device.type == "cuda" and self.device_bookkeeping:
            db = _DeviceBatch(self, seqs)
        # all host-built metadata of the step (batch layout and sampling inputs) in one transfer
        finish_batch = self.prepare_full(seqs) if is_full else self.prepare_sparse(seqs)
        pruned = not is_full and all(q_pruned_step(s, self.config.refresh_period) for s in seqs)
        self.num_q_pruned_forwards += int(pruned)
        finish_sample = self.prepare_sample(seqs, pruned)
        staged = self.staging.flush()
        input_ids, positions = finish_batch(staged)
        params, indices, transfers = finish_sample(staged)
        logits = self.run_model(input_ids, positions, is_full)
        with torch.inference_mode():
            pos, tok, cnt = self.sampler(input_logits=logits, ctx=get_context(), input_indices=indices,
                                         temperatures=params[0], num_transfer=transfers, top_k=params[1],
                                         top_p=params[2], block_size=params[3], confidence_thresholds=params[4])
        reset_context()
        if db is not None:
            db.record(pos, tok, cnt)
            self._dev_batch = db
        return pos, tok, cnt

    def call(self, method: str, *args):
        return getattr(self, method)(*args)

    def exit(self):
        pass
