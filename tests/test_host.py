"""Host-side checks that need no GPU: the C ABI library, the call surface, layouts, schedule."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from resihp import _hip
from resihp.config import TrainConfig
from resihp.model import MLP_RATIO, CausalSelfAttention, ReferenceTransformer
from resihp.parallel import reshard
from resihp.parallel.tp import TensorParallelStage
from resihp.planner.pp import balanced_layers, peak_in_flight, pipeline_phases, pipeline_schedule

HEADER = Path(__file__).resolve().parents[1] / "include" / "resihp_hip.h"

CONFIG = TrainConfig(model_dim=16, num_layers=4, num_heads=4, batch_size=4, micro_batch_size=2, seed=1234,
                     tp=2, pp=2, dp=2, iterations=3)


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int)\s+(rh_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_entry_point():
    lib = _hip.load()
    declared = _declared()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_hip.EXPORTED)


def test_library_version_and_argument_errors():
    lib = _hip.load()
    assert lib.rh_version() == 100
    desc = _hip.rh_gemm_desc()
    desc.dtype = 7
    with pytest.raises(ValueError, match="unknown dtype"):
        _hip.call("rh_gemm", ctypes.byref(desc), None, 0, None)
    desc.dtype = _hip.RH_DTYPE_BF16
    desc.layout = 9
    with pytest.raises(ValueError, match="unknown layout"):
        _hip.call("rh_gemm", ctypes.byref(desc), None, 0, None)
    with pytest.raises(ValueError, match="head_dim"):
        _hip.call("rh_attn_fwd", 1, 1, 8, 1, 256, None, None, None, 256, None, None, 256, None, 1.0, 1, None)
    with pytest.raises(ValueError, match="shard_dim"):
        ext = (ctypes.c_int64 * 1)(4)
        _hip.call("rh_reshard_pack", (ctypes.c_void_p * 1)(None), ext, 1, 4, 4, 2, 2, None, None)
    with pytest.raises(ValueError, match="dim"):
        _hip.call("rh_layernorm_fwd", 0, 4, 0, None, None, None, 1e-5, None, None, None, None)


def test_gemm_kernel_name_reports_the_planned_instantiation():
    """Planning needs no GPU (an absent device counts as 256 CUs): the wgrad of the 1.3B shard's
    fc layers is a split-K direct-to-LDS TN GEMM (split slices run on the 4-wave 256x256 tile, unsplit
    single GEMMs on the 8-wave one), a ragged fp32 GEMM the FMA kernel."""
    def name(dtype, layout, M, N, K, align=16, lda=None):
        d = _hip.rh_gemm_desc()
        d.dtype, d.layout, d.M, d.N, d.K = dtype, layout, M, N, K
        d.b_nseg = d.d_nseg = 1
        d.A, d.B[0], d.D[0] = 0x10000, 0x20000 + align % 16, 0x30000
        d.lda = lda or (M if layout == _hip.RH_GEMM_TN else K)
        d.ldb = K if layout == _hip.RH_GEMM_NT else N
        d.ldd = N
        d.alpha = 1.0
        buf = ctypes.create_string_buffer(128)
        _hip.call("rh_gemm_kernel_name", ctypes.byref(d), buf, 128)
        return buf.value.decode()

    assert name(_hip.RH_DTYPE_BF16, _hip.RH_GEMM_TN, 2048, 2048, 8192) == "gemm_bf16_dma<256, 256, 2, 2, 2, 0, true>"
    assert name(_hip.RH_DTYPE_BF16, _hip.RH_GEMM_NT, 8192, 2048, 2048) == "gemm_bf16_dma<256, 256, 2, 4, 0, 0, false>"
    # N = 1536 (the q|k|v projection): 256x192 tiles, exactly one per CU
    assert name(_hip.RH_DTYPE_BF16, _hip.RH_GEMM_NT, 8192, 1536, 2048) == "gemm_bf16_dma<256, 192, 4, 2, 0, 0, false>"
    assert name(_hip.RH_DTYPE_BF16, _hip.RH_GEMM_NN, 8192, 1536, 2048).startswith("gemm_bf16_dma<256, ")
    # ragged K (LM head dgrad, K = vocab 50257, logits rows padded to 50264): the 64-aligned bulk
    # on the direct-to-LDS kernel
    assert name(_hip.RH_DTYPE_BF16, _hip.RH_GEMM_NN, 8192, 768, 50257, lda=50264).startswith("gemm_bf16_dma<")
    assert name(_hip.RH_DTYPE_BF16, _hip.RH_GEMM_NT, 8192, 2048, 2048, align=2).startswith("gemm_bf16_mfma<")
    assert name(_hip.RH_DTYPE_F32, _hip.RH_GEMM_NN, 100, 77, 50) == "gemm_f32_fma<1, 0, false>"


def test_gemm_descriptor_layout_matches_the_header():
    # int32 x6, then int64 M/N/K at offset 24; pointer arrays of RH_MAX_SEG
    assert _hip.rh_gemm_desc.M.offset == 24
    assert _hip.rh_gemm_desc.B.size == 8 * _hip.RH_MAX_SEG
    assert ctypes.sizeof(_hip.rh_gemm_desc) == 24 + 3 * 8 + 8 + 8 + 32 + 8 + 8 + 8 + 8 + 8 + 32 + 8 + 8 + 8 + 8 + 8


def _expected_names(num_layers):
    names = {"token_embedding.weight", "position_embedding.weight", "final_norm.weight", "final_norm.bias",
             "lm_head.weight"}
    for gid in range(num_layers):
        for suffix in ("attn_norm.weight", "attn_norm.bias", "attn.q_proj.weight", "attn.k_proj.weight",
                       "attn.v_proj.weight", "attn.out_proj.weight", "mlp_norm.weight", "mlp_norm.bias",
                       "mlp.fc1.weight", "mlp.fc2.weight"):
            names.add(f"layers.{gid}.{suffix}")
    return names


def test_model_names_ids_count_and_live_references():
    model = ReferenceTransformer(CONFIG, vocab_size=32, sequence_length=8)
    assert model.layer_ids == (0, 1, 2, 3)
    state = model.logical_state_dict()
    assert set(state) == _expected_names(4)
    params = dict(model.named_parameters())
    assert all(state[n] is params[n] for n in state)
    layer0 = sum(t.numel() for n, t in state.items() if n.startswith("layers.0."))
    assert layer0 == 12 * 16**2 + 4 * 16
    assert MLP_RATIO == 4
    assert state["layers.0.mlp.fc1.weight"].shape == (64, 16)


def test_indivisible_heads_rejected():
    with pytest.raises(ValueError):
        CausalSelfAttention(10, 4)


def test_cpu_forward_fails_loudly():
    model = ReferenceTransformer(CONFIG, vocab_size=32, sequence_length=8)
    with pytest.raises(RuntimeError, match="GPU"):
        model(torch.zeros(2, 8, dtype=torch.int64))
    with pytest.raises(ValueError):
        model(torch.zeros(2, 7, dtype=torch.int64))


def test_stage_layout_matches_shard_dims():
    layer_ids = range(3)
    layout = reshard.shard_dims(layer_ids)
    torch.manual_seed(7)
    ref = ReferenceTransformer(TrainConfig(model_dim=16, num_layers=3, num_heads=4, batch_size=4,
                                           micro_batch_size=2, seed=7, tp=1, pp=1, dp=1, iterations=1),
                               vocab_size=32, sequence_length=8)
    full = ref.logical_state_dict()
    local = {n: torch.chunk(full[n], 2, d)[1].contiguous() if d is not None else full[n].detach()
             for n, d in layout.items()}
    stage = TensorParallelStage(ref.config, vocab_size=32, sequence_length=8, layer_ids=layer_ids, is_first=True,
                                is_last=True, local_state=local, tp_rank=1, tp_size=2)
    assert {n: d for n, (_, d) in stage.local_shards().items()} == layout
    assert stage.vocab_start == 16 and stage.vocab_per_rank == 16
    assert stage.blocks["0"].q_proj.shape == (8, 16) and stage.blocks["0"].out_proj.shape == (16, 8)


def test_stage_rejects_indivisible_degree_and_multi_rank_groups(monkeypatch):
    with pytest.raises(ValueError):
        TensorParallelStage(CONFIG, vocab_size=30, sequence_length=8, layer_ids=[0], is_first=False, is_last=False,
                            local_state={}, tp_rank=0, tp_size=4)
    import torch.distributed as dist

    monkeypatch.setattr(dist, "is_initialized", lambda: True)
    monkeypatch.setattr(dist, "get_world_size", lambda group=None: 2)
    monkeypatch.setattr(dist, "get_rank", lambda group=None: 0)
    with pytest.raises(NotImplementedError):
        TensorParallelStage(CONFIG, vocab_size=32, sequence_length=8, layer_ids=[], is_first=False, is_last=False,
                            local_state={})


@pytest.mark.parametrize("size", [0, 1, 2, 3, 5, 7, 8, 10, 13, 16, 2048])
@pytest.mark.parametrize("parts", [1, 2, 3, 4, 8])
def test_chunk_bounds_follow_torch_chunk(size, parts):
    pieces = torch.chunk(torch.arange(size), parts)
    bounds = reshard._chunk_bounds(size, parts)
    if size:
        assert len(bounds) == len(pieces)
        for (lo, hi), piece in zip(bounds, pieces):
            assert piece.tolist() == list(range(lo, hi))


def test_reconstruct_full_fallbacks_on_cpu():
    a = torch.arange(6.0).reshape(2, 3)
    ckpt = torch.zeros(2, 6)
    full, source = reshard.reconstruct_full("w", 1, 2, {0: a}, checkpoint={"w": ckpt})
    assert source == "checkpoint" and full is ckpt
    with pytest.raises(reshard.ReshardError):
        reshard.reconstruct_full("w", 1, 2, {0: a}, checkpoint=None)
    one = torch.ones(3)
    full, source = reshard.reconstruct_full("n", None, 2, {1: one})
    assert source == "peer" and full is one


def test_schedule_functions():
    assert balanced_layers(5, 2) == ((0, 1, 2), (3, 4))
    assert pipeline_phases(4, stage_index=0, num_stages=2) == (1, 3)
    assert pipeline_schedule(4, stage_index=1, num_stages=2) == ("F", "B") * 4
    assert [peak_in_flight(4, stage_index=i, num_stages=3) for i in range(3)] == [3, 2, 1]
    assert [peak_in_flight(2, stage_index=i, num_stages=4) for i in range(4)] == [2, 2, 2, 1]
    assert peak_in_flight(8, stage_index=1, num_stages=4) == 3
    for bad in ((4, 2, 2), (4, -1, 2), (4, 0, 0)):
        with pytest.raises(ValueError):
            pipeline_phases(bad[0], stage_index=bad[1], num_stages=bad[2])
    with pytest.raises(ValueError):
        pipeline_phases(-1, stage_index=0, num_stages=1)


def test_profiling_short_name_strips_namespaces_and_parameters():
    from resihp.profiling import _short_name

    full = "void rh_gemm_impl::gemm_bf16_dma<256, 256, 2, 4, 2, 0, true>(rh_gemm_impl::GemmParams<unsigned short>)"
    assert _short_name(full) == "gemm_bf16_dma<256, 256, 2, 4, 2, 0, true>"
    anon = "void (anonymous namespace)::attn_fwd_mfma<128>((anonymous namespace)::AttnArgs<unsigned short>, int)"
    assert _short_name(anon) == "attn_fwd_mfma<128>"
    assert _short_name("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"
    # template arguments that name namespaced types are kept whole
    torch_k = "void at::native::vectorized_elementwise_kernel<8, at::native::FillFunctor<float> >(int, float)"
    assert _short_name(torch_k) == "vectorized_elementwise_kernel<8, at::native::FillFunctor<float> >"


def test_1f1b_refuses_a_vocab_parallel_last_stage():
    """A last stage with tp_size > 1 holds only its vocabulary slice of the logits; the reference
    scores the all-gathered logits (parallel/pp.py:375-384), so run_1f1b refuses instead of
    computing a cross-entropy over the slice."""
    from resihp.parallel.pp import run_1f1b

    torch.manual_seed(3)
    ref = ReferenceTransformer(TrainConfig(model_dim=16, num_layers=1, num_heads=4, batch_size=4,
                                           micro_batch_size=2, seed=3, tp=1, pp=1, dp=1, iterations=1),
                               vocab_size=32, sequence_length=8)
    layout = reshard.shard_dims([0])
    full = ref.logical_state_dict()
    local = {n: torch.chunk(full[n], 2, d)[0].contiguous() if d is not None else full[n].detach()
             for n, d in layout.items()}
    stage = TensorParallelStage(ref.config, vocab_size=32, sequence_length=8, layer_ids=[0], is_first=False,
                                is_last=True, local_state=local, tp_rank=0, tp_size=2)
    with pytest.raises(NotImplementedError, match="all-gathered"):
        run_1f1b(stage, stage_index=1, num_stages=2, inputs=[torch.zeros(2, 8, 16)], tokens=[torch.zeros(2, 8)])


# the reference's own routing cases (tests/test_parallel_pp.py:95-101) and properties (:106-141)
_ROUTING_CASES = [((0,), (1,)), ((0, 1), (2, 3)), ((0, 1), (2,)), ((0,), (1, 2)), ((0, 1, 2, 3), (4, 5))]


@pytest.mark.parametrize("up,down", _ROUTING_CASES)
def test_boundary_routing_spreads_one_copy_over_n_links(up, down):
    from resihp.parallel.boundary import scatter_routing

    routing = scatter_routing(up, down)
    chunks = max(len(up), len(down))
    assert len(routing) == chunks and len(set(routing)) == chunks
    for members, end in ((up, 0), (down, 1)):
        runs = [[k for k, pair in enumerate(routing) if pair[end] == m] for m in members]
        assert all(runs)
        for run in runs:
            assert run == list(range(run[0], run[0] + len(run))) and len(run) == chunks // len(members)
        assert [k for run in runs for k in run] == list(range(chunks))


def test_boundary_chunks_and_send_views():
    from resihp.parallel.boundary import my_chunks, scatter_routing, scatter_send_chunks

    assert scatter_routing((0, 1, 2, 3), (4, 5)) == ((0, 4), (1, 4), (2, 5), (3, 5))
    assert my_chunks(4, (0, 1, 2, 3), (4, 5)) == ((0, 0), (1, 1))
    assert my_chunks(2, (0, 1, 2, 3), (4, 5)) == ((2, 5),)
    assert my_chunks(0, (0,), (1, 2)) == ((0, 1), (1, 2))
    with pytest.raises(ValueError):
        my_chunks(9, (0,), (1,))
    t = torch.arange(24.0).reshape(2, 3, 4)
    sends = scatter_send_chunks(t, 0, (0,), (1, 2))
    assert [p for p, _ in sends] == [1, 2]
    assert torch.equal(torch.cat([c for _, c in sends]), t.reshape(-1))
    assert sends[1][1].data_ptr() == t.reshape(-1)[12:].data_ptr()  # a view, not a copy
    with pytest.raises(ValueError, match="equal chunks"):
        scatter_send_chunks(torch.zeros(5), 0, (0,), (1, 2))
