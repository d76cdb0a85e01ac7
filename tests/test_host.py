"""CPU-side checks of the host layer: the C-ABI library loads and exports every symbol the
header declares (no compute call needs a GPU here), the ctypes table matches the header,
argument validation raises like the reference's TORCH_CHECKs, and host bookkeeping."""
import os
import re
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dyllm_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dyllm_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from dyllm_amd import _lib

    lib = _lib.load()
    names = _declared()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/dyllm_hip.h but not exported"
    assert lib.dyllm_abi_version() == 5


def _ctype_of(param):
    import ctypes

    decl = param.strip()
    if "*" in decl:
        return ctypes.c_void_p
    ty = decl.rsplit(" ", 1)[0].replace("const ", "").strip()
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t,
            "float": ctypes.c_float, "uint32_t": ctypes.c_uint32}[ty]


def test_ctypes_table_matches_header():
    from dyllm_amd import _lib

    assert set(_lib.SIGNATURES) == set(_declared())
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, args in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), f"{name}: header has {len(params)} params, ctypes {len(args)}"
        # every parameter's ctypes type matches its C type: a pointer bound as an int (or the
        # reverse) truncates addresses and makes kernels write to wild memory
        for p, a in zip(params, args):
            want = _ctype_of(p)
            assert a is want, f"{name}: parameter '{p.strip()}' is bound as {a.__name__}, header type needs {want.__name__}"


def test_error_path_reports_message_without_gpu():
    """A call that fails validation returns a status and a message, before any launch."""
    from dyllm_amd import _lib

    with pytest.raises(RuntimeError, match="supported head dimension is 128"):
        _lib.call("dyllm_flash_attn_varlen", 1, 1, 1, 1, 1, 4, 4, 64, 1, 1, None, 8, 8, 1.0, None, None)
    with pytest.raises(RuntimeError, match="query heads must be a positive multiple"):
        _lib.call("dyllm_attention_sparse_varlen", 1, 1, 1, 1, 1, 1, 1, 6, 4, 128, 1, 1, 8, 8, 8, 0, 1, None, None,
                  1, 1, 0.99, 1, 1 << 20, None)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _lib.call("dyllm_attention_sparse_varlen", 1, 1, 1, 1, 1, 1, 1, 4, 4, 128, 1, 1, 8, 8, 8, 0, 1, None, None,
                  1, 1, 0.99, 1, 16, None)
    with pytest.raises(RuntimeError, match="hidden size must be a positive multiple of 64"):
        _lib.call("dyllm_ffn_gate_up", 1, 100, None, 10, None, 0, 1, 100, 128, 1, None)
    with pytest.raises(RuntimeError, match="must not be NULL"):
        _lib.call("dyllm_get_seqs", 1, 1, 16, None, 1, 1, 1, 4, None)
    # misaligned buffers are refused before any launch (the kernels use 16-byte accesses)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        _lib.call("dyllm_rms_norm", 2, 4096, None, 0, 16, 10, 4096, 1e-6, 32, 4096, None, 0, None)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        _lib.call("dyllm_linear", 8, 4096, None, 10, None, 0, 16, 8192, 4096, None, 32, None, 0, None)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        _lib.call("dyllm_kv_rope_scatter", 4, 8192, 10, None, None, 16, 16, 16, 4096, 32, 128, None, 1e-6, 16, 16,
                  16, 16, 16, 1, 16, None)
    lib = _lib.load()
    assert lib.dyllm_swiglu_ffn_workspace_bytes(920, 12288) >= 920 * 12288 * 2
    assert lib.dyllm_attention_sparse_workspace_bytes(8, 32, 6144, 1024) >= 6144 * 4 + 32 * 3 * 6144 * 4


def test_ops_validate_like_torch_check():
    from dyllm_amd import ops

    q = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ops.flash_attn_varlen_func(q, q, q, torch.tensor([0, 4]), torch.tensor([0, 4]), 4, 4)
    with pytest.raises(RuntimeError, match="non-causal"):
        ops.flash_attn_varlen_func(q, q, q, torch.tensor([0, 4]), torch.tensor([0, 4]), 4, 4, causal=True)


def test_cache_manager_host_bookkeeping():
    """Slab allocation, contiguity detection and removal, on CPU tensors (no kernel call)."""
    from dyllm_amd.engine.cache_manager import CacheManager

    cm = CacheManager(8, max_num_seqs=16, dtype=torch.float32, device=torch.device("cpu"))
    cm._vectorized_allocate_new_seqs([3, 5, 1], [10, 4, 6])
    assert cm._seq_to_start == {3: 0, 5: 10, 1: 14} and cm.cache.shape == (20, 8)
    assert cm.seq_start_gpu[[3, 5, 1]].tolist() == [0, 10, 14]
    cm._slab[:20] = torch.arange(20, dtype=torch.float32)[:, None]
    view = cm._contiguous_view([3, 5, 1], [0, 10, 14, 20])
    assert view is not None and view.data_ptr() == cm._slab.data_ptr()
    assert cm._contiguous_view([5, 3, 1], [0, 4, 14, 20]) is None  # different order: needs a gather
    cm.remove_seq(5)
    assert cm._seq_to_start == {3: 0, 1: 10} and cm.cache.shape == (16, 8)
    assert cm.seq_start_gpu[1].item() == 10 and cm.seq_start_gpu[5].item() == -1
    assert cm.cache[10:16, 0].tolist() == [14.0, 15.0, 16.0, 17.0, 18.0, 19.0]
    cm._vectorized_allocate_new_seqs([7], [2000])  # grows the slab, keeps the rows
    assert cm._slab.shape[0] >= 2016 and cm.cache[10, 0].item() == 14.0
    assert cm.finish([3, 1, 7]) and cm.num_total_seqs == 0 and cm.cache.shape[0] == 0


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_pinned_salient_count_poll(monkeypatch):
    """Compacted.host() reads the pinned [count, cu_salientlens...] buffer once no entry is
    negative (-1 = not yet written by the compaction kernel), and gives up with an error if the
    kernel never writes it."""
    import torch
    from dyllm_amd import ops

    comp = ops.Compacted(None, None, None, None, None, host_meta=torch.tensor([5, 0, 2, 5], dtype=torch.int32))
    assert comp.host() == (5, [0, 2, 5])
    monkeypatch.setattr(ops, "_HOST_META_TIMEOUT_S", 0.05)
    stale = ops.Compacted(None, None, None, None, None, host_meta=torch.tensor([5, 0, -1, 5], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="not written"):
        stale.host()
    # the compaction's bounded look-back ran out: its count is the failure code, reported at once
    failed = ops.Compacted(None, None, None, None, None, host_meta=torch.tensor([-2, 0, -1, -1], dtype=torch.int32))
    with pytest.raises(RuntimeError, match="look-back"):
        failed.host()


def test_kv_epilogue_struct_matches_header():
    """The ctypes mirror of dyllm_kv_epilogue has the header's fields, in order, with the same
    C types (a mismatch shifts every later field and hands kernels wrong pointers)."""
    import ctypes

    from dyllm_amd import _lib

    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct dyllm_kv_epilogue \{(.*?)\} dyllm_kv_epilogue;", text, flags=re.S).group(1)
    fields = [f.strip() for f in body.split(";") if f.strip()]
    assert len(fields) == len(_lib.KvEpilogue._fields_)
    for decl, (name, ctype) in zip(fields, _lib.KvEpilogue._fields_):
        assert decl.split()[-1].lstrip("*") == name
        assert _ctype_of(decl) is ctype, f"{decl}: bound as {ctype.__name__}"
    assert ctypes.sizeof(_lib.KvEpilogue) == 96
