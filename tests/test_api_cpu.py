"""CPU tests of the host side: the C ABI loads and exports what include/elsa_hip.h
declares, struct layouts match, the planner routes as documented, invalid calls
fail with a status and a message (no GPU needed: no kernel is launched), and the
Python API raises the reference's ValueErrors."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from elsa_amd import _lib
import elsa_amd

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions():
    text = (ROOT / "include" / "elsa_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(elsa_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert set(declared) == set(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_torch_module_loads_with_the_library_abi():
    mod = _lib.torch_module()
    assert mod.abi_version() == _lib.ABI_VERSION
    assert callable(mod.qkv_attention_train) and callable(mod.current_stream)


def test_abi_version_and_struct_sizes():
    lib = _lib.load()
    assert lib.elsa_abi_version() == _lib.ABI_VERSION == 4
    for which, st in _lib._STRUCTS.items():
        assert lib.elsa_struct_size(which) == ctypes.sizeof(st)


def _args(n=16384, bh=(1, 8), d=64, dtype=_lib.ELSA_F16, causal=0, part=0, qc=0):
    a = _lib.FwdArgs()
    a.q = a.k = a.v = a.out = 1
    a.batch, a.heads = bh
    a.seq_len, a.head_dim = n, d
    a.dtype = dtype
    a.summary_dtype = dtype
    a.is_causal = causal
    a.partition_len = part
    a.q_chunk = qc
    return a


def _plan(a):
    lib = _lib.load()
    p = _lib.FwdPlan()
    rc = lib.elsa_fwd_plan_get(ctypes.byref(a), ctypes.byref(p))
    return rc, p


def test_plan_north_star_routing():
    rc, p = _plan(_args())
    assert rc == 0
    assert p.partitions >= 2 and p.partitions * p.partition_len >= 16384
    assert p.q_chunk == 16384 and p.block_m == 256 and p.key_tile == 64
    rows = p.partitions * 8 * 16384
    assert p.workspace_bytes >= rows * (8 + 64 * 2)


@pytest.mark.parametrize("n,dtype,d,causal,parts,part", [
    (4096, _lib.ELSA_F16, 64, 0, 4, 1024),   # the ping-pong fold's partitions of >= 1024 keys
    (4096, _lib.ELSA_BF16, 64, 0, 4, 1024),
    (2048, _lib.ELSA_F16, 64, 0, 4, 512),    # 2K keeps four partitions of 512 (the 4-wave fold)
    (4096, _lib.ELSA_F16, 64, 1, 4, 1024),   # causal: 128-row blocks (a short causal grid), ~1024 workgroups
    (4096, _lib.ELSA_F16, 32, 0, 8, 512),
])
def test_plan_ping_pong_partitions_from_4k(n, dtype, d, causal, parts, part):
    rc, p = _plan(_args(n=n, dtype=dtype, d=d, causal=causal))
    assert rc == 0 and (p.partitions, p.partition_len) == (parts, part)


def _pp_rounds_model(n, bh, q_rows=None):
    """The partition count of the ping-pong routing, restated: the count in [1 or 2, n / 1024] that
    minimises ceil(work-groups / 256) x (partition keys + 768), ties to the fewer."""
    tiles = bh * -(-(q_rows or n) // 512)
    lo = 2 if n >= 8192 else 1
    best = None
    for c in range(lo, max(lo, n // 1024) + 1):
        part = -(-(-(-n // c)) // 64) * 64
        cost = -(-(tiles * -(-n // part)) // 256) * (part + 768)
        if best is None or cost < best[0]:
            best = (cost, part)
    return best[1]


# the ping-pong fold's routing: one round of 512-row work-groups where the grid allows (measured
# bests: B1 H8 8K 2 partitions, B4 H8 4K and B8 H3 N4097 one, B2 H8 N4097 three, B1 H8 N12000 four)
@pytest.mark.parametrize("n,bh,dtype,parts,part", [
    (16384, (1, 8), _lib.ELSA_F16, 2, 8192),   # the north star keeps two
    (8192, (1, 8), _lib.ELSA_F16, 2, 4096),
    (8192, (1, 8), _lib.ELSA_BF16, 2, 4096),
    (4096, (4, 8), _lib.ELSA_F16, 1, 4096),    # one partition (n < 8K): the finalize is fused
    (4097, (8, 3), _lib.ELSA_F16, 1, 4097),
    (4097, (2, 8), _lib.ELSA_F16, 3, 1408),
    (12000, (1, 8), _lib.ELSA_F16, 4, 3008),
    (65536, (1, 8), _lib.ELSA_F16, 2, 32768),
    (16384, (1, 2), _lib.ELSA_F16, 4, 4096),
])
def test_plan_ping_pong_one_round(n, bh, dtype, parts, part):
    rc, p = _plan(_args(n=n, bh=bh, dtype=dtype))
    assert rc == 0 and (p.partitions, p.partition_len) == (parts, part)
    assert min(part, n) == min(_pp_rounds_model(n, bh[0] * bh[1]), n)


def test_plan_ping_pong_rule_only_where_the_ping_pong_fold_runs():
    # fp16 inputs with fp32 summaries run the 4-wave fold (p unrounded for P.V): ~1024 256-row work-groups
    a = _args(n=8192)
    a.summary_dtype = _lib.ELSA_F32
    rc, p = _plan(a)
    assert rc == 0 and (p.partitions, p.partition_len) == (4, 2048)
    # fp32 and d128 (128-row blocks, 512 of them at B1 H8 8K): two partitions of the 1024 target
    rc, p = _plan(_args(n=8192, dtype=_lib.ELSA_F32))
    assert rc == 0 and (p.block_m, p.partitions) == (128, 2)
    rc, p = _plan(_args(n=8192, d=128))
    assert rc == 0 and (p.block_m, p.partitions) == (128, 2)
    rc, p = _plan(_args(n=8192, bh=(1, 2), d=32))  # the 4-wave fold at d32: 1024 / 64 = 16 of 512 keys
    assert rc == 0 and (p.partitions, p.partition_len) == (16, 512)


# fp32 grids the 1024-workgroup rule leaves under 256 work-groups take partitions down to 64 keys
# until about 512 (measured: B1 H8 1K 0.050 -> 0.029 ms, B8 H3 N197 0.024 -> 0.013 ms); larger ones keep it
@pytest.mark.parametrize("n,bh,causal,parts,part", [
    (1024, (1, 8), 0, 8, 128), (1024, (1, 8), 1, 8, 128), (512, (1, 8), 0, 8, 64),
    (197, (8, 3), 0, 4, 64),     # ceil(197 / 64) partitions: two stages per work-group, not three
    (90, (1, 2), 0, 2, 64),
    (1024, (2, 8), 1, 4, 256),   # causal: filled below 512 work-groups (half of them return at once)
    (1024, (2, 8), 0, 2, 512),   # non-causal: 256 work-groups already
    (1025, (8, 3), 0, 2, 544),   # 432 work-groups already: two partitions (0.086 against 0.089 ms with three)
    (2048, (1, 8), 0, 4, 512), (4096, (1, 8), 0, 4, 1024),
])
def test_plan_fp32_fills_short_grids(n, bh, causal, parts, part):
    rc, p = _plan(_args(n=n, bh=bh, dtype=_lib.ELSA_F32, causal=causal))
    assert rc == 0 and (p.partitions, p.partition_len) == (parts, part) and p.block_m == 128


# fp16/bf16 at d <= 64 under 192 work-groups: partitions down to 128 keys until about 256 work-groups
@pytest.mark.parametrize("n,bh,dtype,causal,parts,part", [
    (1024, (1, 8), _lib.ELSA_F16, 0, 4, 256), (1024, (1, 8), _lib.ELSA_BF16, 0, 4, 256),
    (512, (1, 8), _lib.ELSA_F16, 0, 4, 128),
    (197, (8, 3), _lib.ELSA_F16, 0, 1, 197),    # ViT-T 224 px keeps its one fused partition
    (1025, (8, 3), _lib.ELSA_F16, 0, 2, 576),   # 240 work-groups: unchanged
    (2048, (1, 8), _lib.ELSA_F16, 0, 4, 512),
])
def test_plan_short_16bit_grids_fill_to_256(n, bh, dtype, causal, parts, part):
    rc, p = _plan(_args(n=n, bh=bh, dtype=dtype, causal=causal))
    assert rc == 0 and (p.partitions, p.partition_len) == (parts, part)


@pytest.mark.parametrize("n,bh,d", [(49, (8, 3), 32), (197, (8, 3), 64), (1024, (1, 8), 64), (65536, (1, 8), 64),
                                    (4097, (8, 3), 64), (300, (1, 2), 128)])
def test_plan_partitions_cover_sequence(n, bh, d):
    rc, p = _plan(_args(n=n, bh=bh, d=d))
    assert rc == 0
    assert p.partitions * p.partition_len >= n > (p.partitions - 1) * p.partition_len
    assert p.q_chunk >= 1


@pytest.mark.parametrize("n,part,parts", [(8192, 2048, 4), (16384, 4096, 4), (32768, 8192, 4), (65536, 8192, 8),
                                          (12000, 3072, 4)])
def test_plan_causal_partitions_of_a_quarter_within_2k_8k_from_8k(n, part, parts):
    rc, p = _plan(_args(n=n, causal=1))
    assert rc == 0 and p.partition_len == part and p.partitions == parts
    assert p.partition_len % p.block_m == 0  # whole row blocks: Phase 1 dispatches longest first


def test_plan_causal_short_partitions_round_to_the_nearest_row_block():
    # B1 H8 causal 1025: a short grid (72 row blocks) takes 4 partitions of ceil(1025 / 4) = 257 keys,
    # rounded to the nearest 128-row block: 256 keys, so 5 partitions, the last of one key
    rc, p = _plan(_args(n=1025, causal=1))
    assert rc == 0 and p.block_m == 128 and p.partition_len == 256 and p.partitions == 5
    rc, p = _plan(_args(n=1025, bh=(8, 3), causal=1))  # 216 row blocks: 2 partitions of 513 -> 512
    assert rc == 0 and p.block_m == 128 and p.partition_len == 512 and p.partitions == 3


@pytest.mark.parametrize("n,bh,bm", [(2048, (1, 8), 128), (4097, (1, 8), 128), (1025, (8, 3), 128),
                                     (8192, (1, 8), 256), (4097, (8, 3), 256), (32768, (1, 8), 256)])
def test_plan_causal_block_m_by_grid_size(n, bh, bm):
    # 128-row blocks while the 256-row grid has fewer than 256 (row block, head) pairs
    rc, p = _plan(_args(n=n, bh=bh, causal=1))
    assert rc == 0 and p.block_m == bm
    assert p.partitions == 1 or p.partition_len % p.block_m == 0
    rc, p = _plan(_args(n=n, bh=bh))
    assert rc == 0 and p.block_m == 256  # non-causal calls keep 256 rows above 1024 tokens


@pytest.mark.parametrize("n,d", [(300, 128), (197, 64), (49, 32)])
def test_plan_causal_single_partition_stays_whole(n, d):
    rc, p = _plan(_args(n=n, bh=(2, 2), d=d, causal=1))
    assert rc == 0 and p.partitions == 1 and p.partition_len == n


def test_plan_causal_short_sequences_keep_the_workgroup_target():
    rc_c, pc = _plan(_args(n=2048, causal=1))
    rc_n, pn = _plan(_args(n=2048))
    assert rc_c == rc_n == 0 and pc.partition_len == pn.partition_len == 512


@pytest.mark.parametrize("n,d,dtype,bm", [(49, 32, _lib.ELSA_F16, 64), (197, 64, _lib.ELSA_F16, 128),
                                         (1024, 64, _lib.ELSA_BF16, 128), (1025, 64, _lib.ELSA_F16, 256),
                                         (16384, 64, _lib.ELSA_F16, 256), (4096, 128, _lib.ELSA_F16, 128),
                                         (4096, 64, _lib.ELSA_F32, 128), (64, 64, _lib.ELSA_F32, 64)])
def test_plan_block_m_by_sequence_length(n, d, dtype, bm):
    rc, p = _plan(_args(n=n, d=d, dtype=dtype))
    assert rc == 0 and p.block_m == bm


def test_plan_block_m_with_bias():
    a = _args(n=16384)
    bias = torch.zeros(1)  # only the pointer's presence matters to the planner
    a.bias = _lib.bias_desc(bias, (0, 0, 16384, 1))
    rc, p = _plan(a)
    assert rc == 0 and p.block_m == 128
    a = _args(n=49, d=32)
    a.bias = _lib.bias_desc(bias, (0, 0, 49, 1))
    rc, p = _plan(a)
    assert rc == 0 and p.block_m == 64


def test_plan_user_partition_and_chunk():
    rc, p = _plan(_args(n=513, bh=(1, 2), part=128, qc=128))
    assert rc == 0 and p.partition_len == 128 and p.partitions == 5 and p.q_chunk == 128


@pytest.mark.parametrize("field,value,code", [("head_dim", 136, -1), ("head_dim", 20, -1), ("seq_len", 0, -1),
                                              ("dtype", 7, -1), ("summary_dtype", 9, -1)])
def test_plan_rejects_invalid(field, value, code):
    a = _args()
    setattr(a, field, value)
    rc, _ = _plan(a)
    assert rc == code
    assert _lib.load().elsa_last_error().decode()


def test_fwd_rejects_missing_workspace_without_launching():
    lib = _lib.load()
    a = _args(n=256, bh=(1, 1))
    rc = lib.elsa_fwd(ctypes.byref(a), None)
    assert rc == _lib.ELSA_ERR_WORKSPACE
    assert "workspace" in lib.elsa_last_error().decode()
    a.q = None
    assert lib.elsa_fwd(ctypes.byref(a), None) == _lib.ELSA_ERR_INVALID


def test_fwd_noalloc_rejects_rows_beyond_its_scratch_without_launching():
    """elsa_fwd_noalloc (summaries in the library's 64 MiB device array) refuses a call of which
    a single query row needs more than the array, before any HIP call."""
    lib = _lib.load()
    a = _args(n=8192, bh=(64, 64), part=64)  # 128 partitions x 4096 heads x 136 B = 71 MB per row
    a.q = a.k = a.v = a.out = 1 << 12
    rc = lib.elsa_fwd_noalloc(ctypes.byref(a), None)
    assert rc == _lib.ELSA_ERR_WORKSPACE
    msg = lib.elsa_last_error().decode()
    assert "elsa_fwd_noalloc" in msg and "scratch" in msg
    a.q = None
    assert lib.elsa_fwd_noalloc(ctypes.byref(a), None) == _lib.ELSA_ERR_INVALID


def test_library_imports_no_device_allocation():
    """No entry point of libelsa_hip.so can allocate or free device memory: the library does not
    import any HIP allocation or release routine (callers bring every buffer, elsa_fwd_noalloc
    uses the library's own device array)."""
    import subprocess

    syms = subprocess.run(["nm", "-D", "--undefined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                          check=True).stdout
    hip = sorted({line.split()[-1].split("@")[0] for line in syms.splitlines() if "hip" in line})
    assert hip and not [s for s in hip if re.search(r"(?i)alloc|free|mempool|hostregister", s)], hip


def test_bwd_and_dbias_reject_bad_args_without_launching():
    lib = _lib.load()
    b = _lib.BwdArgs()
    b.batch, b.heads, b.seq_len, b.head_dim, b.dtype = 1, 1, 64, 64, _lib.ELSA_F16
    b.q = b.k = b.v = 256
    assert lib.elsa_bwd(ctypes.byref(b), None) == _lib.ELSA_ERR_INVALID  # no out/dout/grads
    b.out = b.dout = b.dq = b.dk = b.dv = b.row_m = b.row_z = 256
    assert lib.elsa_bwd(ctypes.byref(b), None) == _lib.ELSA_ERR_WORKSPACE
    assert lib.elsa_bwd_workspace_bytes(ctypes.byref(b)) >= 2 * 64 * 4
    assert lib.elsa_dbias_workspace_bytes(ctypes.byref(b), 1, 1) >= lib.elsa_bwd_workspace_bytes(ctypes.byref(b))
    assert lib.elsa_dbias_workspace_bytes(ctypes.byref(b), 0, 1) == 0
    assert lib.elsa_dbias(ctypes.byref(b), 1, 2, 1, None) == _lib.ELSA_ERR_INVALID  # bias_batch 2 vs B=1
    assert lib.elsa_debug_mfma(5, 1, 1, 1, None) == _lib.ELSA_ERR_INVALID
    assert lib.elsa_debug_mfma_rate(3, 1, 1, 10, 1, None) == _lib.ELSA_ERR_INVALID
    assert lib.elsa_debug_mfma_rate(0, 1, 1, 0, 1, None) == _lib.ELSA_ERR_INVALID
    assert lib.elsa_debug_mfma_rate(0, 1, 1, 10, 0, None) == _lib.ELSA_ERR_INVALID
    assert lib.elsa_debug_mfma_rate(0, None, 1, 10, 1, None) == _lib.ELSA_ERR_INVALID
    assert lib.elsa_debug_mfma_rate(0, 1, 1, 1000000, 65536, None) == _lib.ELSA_ERR_INVALID  # launch too long


def test_bwd_dbias_rejects_bad_args_and_sizes_its_workspace():
    lib = _lib.load()
    b = _lib.BwdArgs()
    b.batch, b.heads, b.seq_len, b.head_dim, b.dtype = 2, 3, 64, 64, _lib.ELSA_F16
    b.q = b.k = b.v = b.out = b.dout = b.dq = b.dk = b.dv = b.row_m = b.row_z = 256
    rows = lib.elsa_bwd_workspace_bytes(ctypes.byref(b))
    ds = 2 * 3 * 64 * 64 * 4
    # dbias of the bias's own shape is dS itself; a broadcast bias needs the dS buffer
    assert lib.elsa_bwd_dbias_workspace_bytes(ctypes.byref(b), 2, 3) == rows
    assert lib.elsa_bwd_dbias_workspace_bytes(ctypes.byref(b), 1, 3) == rows + ds
    assert lib.elsa_bwd_dbias(ctypes.byref(b), 256, 2, 3, None) == _lib.ELSA_ERR_INVALID  # no bias
    assert "bias" in lib.elsa_last_error().decode()
    bias = torch.zeros(1)
    b.bias = _lib.bias_desc(bias, (0, 64 * 64, 64, 1))
    assert lib.elsa_bwd_dbias(ctypes.byref(b), 256, 3, 3, None) == _lib.ELSA_ERR_INVALID  # 3 does not broadcast to 2
    assert lib.elsa_bwd_dbias(ctypes.byref(b), 256, 1, 3, None) == _lib.ELSA_ERR_WORKSPACE
    assert lib.elsa_bwd_dbias(ctypes.byref(b), None, 1, 3, None) == _lib.ELSA_ERR_INVALID


def test_bwd_layout_rules_without_launching():
    lib = _lib.load()
    b = _lib.BwdArgs()
    b.batch, b.heads, b.seq_len, b.head_dim, b.dtype = 2, 3, 64, 64, _lib.ELSA_F16
    b.q = b.k = b.v = b.out = b.dout = b.dq = b.dk = b.dv = b.row_m = b.row_z = 256
    b.workspace, b.workspace_bytes = 256, 1 << 20  # never dereferenced: no kernel is launched
    # a [B,N,3,H,D] view (row stride 3*H*D, head stride D) is a valid input and output layout
    b.q_layout = _lib.Layout(64 * 3 * 3 * 64, 64, 3 * 3 * 64)
    b.dq_layout = _lib.Layout(64 * 3 * 3 * 64, 64, 3 * 3 * 64)
    assert lib.elsa_bwd_stage(ctypes.byref(b), 7, None) == _lib.ELSA_ERR_INVALID  # past the layout checks
    assert "stage" in lib.elsa_last_error().decode()
    b.k = 258  # misaligned base
    assert lib.elsa_bwd(ctypes.byref(b), None) == _lib.ELSA_ERR_INVALID
    assert "16-byte" in lib.elsa_last_error().decode()
    b.k = 256
    b.v_layout = _lib.Layout(3 * 64 * 64, 64 * 64, 60)  # row stride < head_dim
    assert lib.elsa_bwd(ctypes.byref(b), None) == _lib.ELSA_ERR_INVALID
    assert "row stride" in lib.elsa_last_error().decode()
    b.v_layout = _lib.Layout(0, 0, 0)
    b.dk_layout = _lib.Layout(3 * 64 * 64, 0, 64)  # heads of an output would share rows
    assert lib.elsa_bwd(ctypes.byref(b), None) == _lib.ELSA_ERR_INVALID
    assert "output" in lib.elsa_last_error().decode()
    b.dk_layout = _lib.Layout(0, 0, 0)
    b.k_layout = _lib.Layout(3 * 64 * 64, 0, 64)  # an input may broadcast over heads
    assert lib.elsa_bwd_stage(ctypes.byref(b), 7, None) == _lib.ELSA_ERR_INVALID
    assert "stage" in lib.elsa_last_error().decode()


def test_python_api_validation_on_cpu_tensors():
    q = torch.zeros(1, 2, 8, 16)
    with pytest.raises(ValueError, match="CUDA"):
        elsa_amd.twopass_attention(q, q, q)
    with pytest.raises(ValueError, match=r"\[B,H,N,D\]"):
        elsa_amd.twopass_attention(q[0], q[0], q[0])
    with pytest.raises(ValueError, match="identical shapes"):
        elsa_amd.twopass_attention(q, q[:, :1], q)
    with pytest.raises(ValueError, match="CUDA"):
        elsa_amd.twopass_attention_with_state(q, q, q)
    with pytest.raises(ValueError, match="CUDA"):
        elsa_amd.twopass_attention_backward(q, q, q, q, q)
    with pytest.raises(ValueError, match="identical shapes"):
        elsa_amd.twopass_attention_backward(q, q, q, q, q[:, :1])


def test_user_tiles_and_warps_validation():
    from elsa_amd.attention import _user_tiles, _validate_warps

    kw = dict(block_m=None, block_n=None, q_chunk_size=None, phase1_warps=None, phase2_warps=None,
              phase1_stages=None, phase2_stages=None)
    # nothing given: the HIP planner routes
    assert _user_tiles(dtype=torch.float16, head_dim=64, **kw) == (None, None)
    # attention.py:302: q_chunk rounded down to the default block_m (64 for fp16 d <= 64, 32 for
    # fp32 or d > 64), never below it; block_n and q_chunk clamped to >= 16 (:228-236)
    assert _user_tiles(dtype=torch.float16, head_dim=64, **dict(kw, block_n=8, q_chunk_size=3000)) == (16, 2944)
    assert _user_tiles(dtype=torch.float32, head_dim=64, **dict(kw, q_chunk_size=3000)) == (None, 2976)
    assert _user_tiles(dtype=torch.float16, head_dim=128, **dict(kw, q_chunk_size=40)) == (None, 32)
    assert _user_tiles(dtype=torch.float16, head_dim=64, **dict(kw, block_m=128, q_chunk_size=300)) == (None, 256)
    with pytest.raises(ValueError, match="1, 2, 4, or 8"):
        _validate_warps("phase1_warps", 3)
    with pytest.raises(ValueError, match="1, 2, 4, or 8"):
        _user_tiles(dtype=torch.float16, head_dim=64, **dict(kw, phase2_warps=16))


def test_canonical_bias_cpu():
    from elsa_amd.attention import _canonical_bias

    dev = torch.device("cpu")
    m = _canonical_bias(torch.zeros(3, 8, 8), batch=2, heads=3, seq_len=8, device=dev)
    assert (m.stride_b, m.stride_h, m.stride_q, m.stride_k) == (0, 64, 8, 1)
    m = _canonical_bias(torch.zeros(8, 8), batch=2, heads=3, seq_len=8, device=dev)
    assert (m.stride_b, m.stride_h) == (0, 0)
    with pytest.raises(ValueError, match="4D bias"):
        _canonical_bias(torch.zeros(3, 3, 8, 8), batch=2, heads=3, seq_len=8, device=dev)
    with pytest.raises(ValueError, match="last dims"):
        _canonical_bias(torch.zeros(8, 7), batch=2, heads=3, seq_len=8, device=dev)


def _align256(x):
    return (x + 255) // 256 * 256


@pytest.mark.parametrize("n,bh,dtype,d,split", [
    (1024, (1, 8), _lib.ELSA_F16, 64, 4),    # 64 four-wave work-groups: four 256-row ranges
    (4096, (1, 8), _lib.ELSA_F16, 64, 2),    # 256 work-groups: two ranges fill the chip twice
    (2048, (1, 8), _lib.ELSA_BF16, 64, 4),
    (1025, (8, 3), _lib.ELSA_F16, 64, 2),    # ViT-T at 512 px: 216 work-groups, doubled once (432)
    (2305, (8, 3), _lib.ELSA_F16, 32, 1),    # 456 work-groups: a doubling would pass one round of 512
    (16384, (1, 8), _lib.ELSA_F16, 64, 1),   # the north star's grid is full
    (197, (8, 3), _lib.ELSA_F16, 64, 1),     # ranges would fall below 256 rows
    (1024, (1, 8), _lib.ELSA_F32, 64, 8),    # fp32 takes 128-row ranges where fp16 stops at 256
    (4096, (1, 8), _lib.ELSA_F32, 64, 2),
    (197, (8, 3), _lib.ELSA_F32, 64, 2),     # fp32 ranges go down to 64 rows: 99 -> two stages of 64
    (512, (1, 8), _lib.ELSA_F32, 64, 8),     # eight 64-row ranges
    (300, (2, 3), _lib.ELSA_F32, 64, 4),     # 75 rows each; eight would fall below 64
    (1024, (1, 8), _lib.ELSA_F16, 128, 1),   # d = 128 keeps its unsplit kernels
])
def test_bwd_workspace_holds_the_split_partials(n, bh, dtype, d, split):
    """Short sequences with few heads cut the backward's key (dq) and row (dK/dV) loops into ranges
    over extra work-groups; the workspace then holds their fp32 partials of dq, dK and dV."""
    lib = _lib.load()
    b = _lib.BwdArgs()
    b.batch, b.heads, b.seq_len, b.head_dim, b.dtype = bh[0], bh[1], n, d, dtype
    rows = bh[0] * bh[1] * n
    part = 3 * _align256(split * rows * d * 4) if split > 1 else 0
    assert lib.elsa_bwd_workspace_bytes(ctypes.byref(b)) == 3 * _align256(rows * 4) + part
    # a bias keeps the unsplit kernels (dS may be stored per score)
    bias = torch.zeros(1)
    b.bias = _lib.bias_desc(bias, (0, 0, n, 1))
    assert lib.elsa_bwd_workspace_bytes(ctypes.byref(b)) == 3 * _align256(rows * 4)


def _causal_live_wgs(bh, n, s):
    # work-groups of a causal fp32 split that hold work: a 128-row block's dq ranges stop at its last
    # row; fp32 ranges are whole 32-key stages
    sl = ((n + s - 1) // s + 31) // 32 * 32
    return bh * sum((min(n, b0 + 128) + sl - 1) // sl for b0 in range(0, n, 128))


@pytest.mark.parametrize("n,bh,dtype,causal,split", [
    (4097, (1, 8), _lib.ELSA_F32, True, 2),    # 264 work-groups, 400 of 528 hold work once doubled
    (2049, (2, 8), _lib.ELSA_F32, True, 2),
    (1025, (1, 8), _lib.ELSA_F32, True, 8),    # 8 ranges of 160 keys: 312 of 576 hold work
    (1025, (1, 8), _lib.ELSA_F32, False, 4),   # non-causal: every work-group counts
    (3000, (1, 8), _lib.ELSA_F32, True, 4),
    (8192, (1, 8), _lib.ELSA_F32, True, 1),    # 512 work-groups fill the round already
    (4097, (1, 8), _lib.ELSA_F16, True, 1),    # 16-bit calls count every work-group
    (2049, (2, 8), _lib.ELSA_BF16, True, 1),
])
def test_causal_fp32_split_counts_the_work_groups_that_hold_work(n, bh, dtype, causal, split):
    """Causal fp32 backward: the split doubles while the work-groups that hold work (the others return
    at once) fit one round of 512; 16-bit and non-causal calls count every work-group."""
    lib = _lib.load()
    b = _lib.BwdArgs()
    b.batch, b.heads, b.seq_len, b.head_dim, b.dtype, b.is_causal = bh[0], bh[1], n, 64, dtype, int(causal)
    rows = bh[0] * bh[1] * n
    part = 3 * _align256(split * rows * 64 * 4) if split > 1 else 0
    assert lib.elsa_bwd_workspace_bytes(ctypes.byref(b)) == 3 * _align256(rows * 4) + part
    if causal and dtype == _lib.ELSA_F32 and split > 1:
        assert _causal_live_wgs(bh[0] * bh[1], n, split) <= 512
        assert split == 8 or n // (2 * split) < 64 or _causal_live_wgs(bh[0] * bh[1], n, 2 * split) > 512
