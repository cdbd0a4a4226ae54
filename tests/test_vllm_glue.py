"""The vLLM installation of runtime.block_view, on stand-ins for the vLLM classes it patches (vLLM is
not installed here): require_supported_attention's refusals (the cases and message fragments of the
reference's tests/test_supported_attention.py), one view per process and cache group, the builders
and attention implementations patched once, a cascade batch skipped, the Triton metadata given the
view's buffers, the audit kernel recording after each layer, and the plane attached by layer name
(runtime/block_view.py:404-626)."""

import enum
import sys
import types
from dataclasses import dataclass, replace
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from runtime import block_view


class AttentionType(str, enum.Enum):
    DECODER = "decoder"
    ENCODER = "encoder"
    ENCODER_ONLY = "encoder_only"


@dataclass
class FullAttentionSpec:
    block_size: int = 16
    sliding_window: int | None = None
    attention_chunk_size: int | None = None


@dataclass
class SlidingWindowSpec(FullAttentionSpec):
    pass


class MambaSpec:
    block_size = 16


class TritonAttentionMetadataBuilder:
    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        return SimpleNamespace(block_table=common_attn_metadata.block_table_tensor,
                               seq_lens=common_attn_metadata.seq_lens)


class FlashInferMetadataBuilder:
    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        return SimpleNamespace(seen=common_attn_metadata)


class TritonAttentionImpl:
    scale = 0.125

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
        return "attended"


class FlashInferImpl(TritonAttentionImpl):
    pass


@pytest.fixture()
def vllm(monkeypatch):
    names = {
        "vllm": {},
        "vllm.v1": {},
        "vllm.v1.attention": {},
        "vllm.v1.attention.backend": {"AttentionType": AttentionType},
        "vllm.v1.kv_cache_interface": {"FullAttentionSpec": FullAttentionSpec,
                                       "SlidingWindowSpec": SlidingWindowSpec, "MambaSpec": MambaSpec},
        "vllm.v1.attention.backends": {},
        "vllm.v1.attention.backends.triton_attn": {"TritonAttentionMetadataBuilder": TritonAttentionMetadataBuilder,
                                                   "TritonAttentionImpl": TritonAttentionImpl},
        "vllm.v1.attention.backends.flashinfer": {"FlashInferMetadataBuilder": FlashInferMetadataBuilder,
                                                  "FlashInferImpl": FlashInferImpl},
    }
    for name, attrs in names.items():
        module = types.ModuleType(name)
        for key, value in attrs.items():
            setattr(module, key, value)
        monkeypatch.setitem(sys.modules, name, module)
    for cls, attr in ((TritonAttentionMetadataBuilder, "build"), (FlashInferMetadataBuilder, "build"),
                      (TritonAttentionImpl, "forward"), (FlashInferImpl, "forward")):
        monkeypatch.setattr(cls, attr, cls.__dict__.get(attr, getattr(cls, attr)))
    monkeypatch.setattr(block_view, "_view", None)
    monkeypatch.setattr(block_view, "_plane", None)
    monkeypatch.setattr(block_view, "_layers", ())
    for var in ("EKV_ATTN_SHARE", "EKV_AUDIT_KERNEL", "EKV_PREFILL_AUDIT"):
        monkeypatch.delenv(var, raising=False)


def layer(sliding_window=None, alibi=None, attn_type=AttentionType.DECODER):
    return SimpleNamespace(sliding_window=sliding_window, impl=SimpleNamespace(alibi_slopes=alibi),
                           attn_type=attn_type)


def builder(spec=None, layers=None, names=("l0", "l1"), rows=2, cls=TritonAttentionMetadataBuilder):
    layers = layers or {name: layer() for name in names}
    b = cls.__new__(cls)
    b.kv_cache_spec = spec or FullAttentionSpec()
    b.layer_names = list(layers)
    b.vllm_config = SimpleNamespace(compilation_config=SimpleNamespace(static_forward_context=layers),
                                    scheduler_config=SimpleNamespace(max_num_seqs=rows))
    return b


@dataclass
class Batch:
    block_table_tensor: torch.Tensor
    seq_lens: torch.Tensor
    query_start_loc_cpu: torch.Tensor
    num_reqs: int
    _seq_lens_cpu: object = None
    max_seq_len: int = 0

    def replace(self, **kw):
        return replace(self, **kw)


def batch(query_lens=(1, 1)):
    starts = torch.tensor(np.concatenate([[0], np.cumsum(query_lens)]), dtype=torch.int32)
    return Batch(torch.zeros(2, 4, dtype=torch.int32), torch.tensor([20, 40], dtype=torch.int32), starts,
                 len(query_lens))


def test_refusals_name_the_cause(vllm):
    block_view.require_supported_attention(builder())
    with pytest.raises(RuntimeError, match="SlidingWindowSpec"):
        block_view.require_supported_attention(builder(SlidingWindowSpec(sliding_window=1024)))
    with pytest.raises(RuntimeError, match="MambaSpec"):
        block_view.require_supported_attention(builder(MambaSpec()))
    for spec in (FullAttentionSpec(sliding_window=512), FullAttentionSpec(attention_chunk_size=256)):
        with pytest.raises(RuntimeError, match="sliding window or chunked"):
            block_view.require_supported_attention(builder(spec))
    with pytest.raises(RuntimeError, match="layer bad has a sliding window"):
        block_view.require_supported_attention(builder(layers={"ok": layer(), "bad": layer(sliding_window=4096)}))
    with pytest.raises(RuntimeError, match="position bias"):
        block_view.require_supported_attention(builder(layers={"bad": layer(alibi=torch.ones(8))}))
    with pytest.raises(RuntimeError, match="encoder"):
        block_view.require_supported_attention(builder(layers={"bad": layer(attn_type=AttentionType.ENCODER)}))


def test_one_view_per_cache_group(vllm):
    first, second = builder(names=("a", "b")), builder(names=("c", "d"))
    view = block_view._view_for(first, batch())
    assert view.rows == 2 and view.width == 4 and view.block_size == 16 and view.audit is None
    assert block_view._view_for(first, batch()) is view
    assert block_view.current_view() is view
    with pytest.raises(RuntimeError, match="several"):
        block_view._view_for(second, batch())


def test_no_view_before_the_first_batch(vllm):
    with pytest.raises(RuntimeError, match="install"):
        block_view.current_view()


def test_both_statistics_at_once_are_refused(vllm, monkeypatch):
    monkeypatch.setenv("EKV_ATTN_SHARE", "1")
    monkeypatch.setenv("EKV_AUDIT_KERNEL", "1")
    with pytest.raises(RuntimeError, match="EKV_ATTN_SHARE"):
        block_view._view_for(builder(), batch())


def test_prefill_audit_needs_the_compiler_pass(vllm, monkeypatch):
    monkeypatch.setenv("EKV_PREFILL_AUDIT", "1")
    with pytest.raises(RuntimeError, match="EKV_ATTN_SHARE"):
        block_view._view_for(builder(), batch())


def test_builders_are_patched_once_and_route_to_the_view(vllm, monkeypatch):
    calls = []
    monkeypatch.setattr(block_view.DecodeView, "build",
                        lambda self, table, lens, q: (calls.append(("build", q.tolist())) or ("view-table", "view-lens")))
    monkeypatch.setattr(block_view.DecodeView, "skip", lambda self, lens, q: calls.append(("skip", q.tolist())))
    assert block_view.install_decode_view() == 2
    assert block_view.install_decode_view() == 0  # already installed
    b = builder()
    metadata = b.build(0, batch((1, 1)))
    assert (metadata.block_table, metadata.seq_lens) == ("view-table", "view-lens")
    metadata = b.build(5, batch((1, 3)))  # a cascade: the engine's own table
    assert metadata.block_table is not None and calls == [("build", [1, 1]), ("skip", [1, 3])]


def test_flashinfer_builds_from_the_view_batch(vllm, monkeypatch):
    lens = torch.tensor([7, 9], dtype=torch.int32)
    monkeypatch.setattr(block_view.DecodeView, "build", lambda self, table, seq, q: ("view-table", lens))
    block_view.install_decode_view()
    out = builder(cls=FlashInferMetadataBuilder).build(0, batch())
    assert out.seen.block_table_tensor == "view-table" and out.seen.seq_lens is lens
    assert out.seen.max_seq_len == 9 and out.seen._seq_lens_cpu is None


def test_the_audit_kernel_records_after_each_layer(vllm, monkeypatch):
    from runtime import audit_kernel

    recorded = []

    class Plane(audit_kernel.RecordingPlane):
        def __init__(self):  # no device: the record call is what is checked
            self._layer_of = {"l0": 0, "l1": 1}

        def record(self, name, table, lens, query, kv_cache, scale):
            recorded.append((name, table, lens, query, kv_cache, scale))

        def attach(self, addresses):
            recorded.append(("attach", addresses))
            return True

    assert block_view.install_audit_kernel() == 2
    assert block_view.install_audit_kernel() == 0
    impl = TritonAttentionImpl()
    assert impl.forward(SimpleNamespace(layer_name="l0"), "q", "k", "v", "cache", None) == "attended"
    assert recorded == []  # a profiling run has no batch
    block_view._view_for(builder(), batch())
    with pytest.raises(RuntimeError, match="recording plane"):
        impl.forward(SimpleNamespace(layer_name="l0"), "q", "k", "v", "cache", object())
    view = block_view.current_view()
    view.audit = Plane()
    view._table, view._lens = "table", "lens"
    assert impl.forward(SimpleNamespace(layer_name="l1"), "q", "k", "v", "cache", object()) == "attended"
    assert recorded == [("l1", "table", "lens", "q", "cache", 0.125)]
    monkeypatch.setattr(block_view, "_plane", view.audit)

    class Cache:
        def __init__(self, address):
            self.address = address

        def data_ptr(self):
            return self.address

    context = {"l0": SimpleNamespace(kv_cache=Cache(100)), "l1": SimpleNamespace(kv_cache=Cache(200))}
    runner = SimpleNamespace(compilation_config=SimpleNamespace(static_forward_context=context))
    assert block_view.attach_audit_plane(runner) is view
    assert recorded[-1] == ("attach", [100, 200])
