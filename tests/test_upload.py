"""Host-side lifecycle of the NF4 staging API on the CPU, covering the behaviours
the reference pins in its own tests (tests/test_upload.py of h4rm0n1c/stratum):
payload survival across parameter replacement, shared-parameter byte estimates,
free_weights scope, empty prefetch, prefetch + ensure chaining, cache v1
accept/reject, FP16-staged lifecycle, 2-D / 3-D prepare with the quantizer
replaced by a recording stand-in, and buffer snapshot/restore."""

from pathlib import Path
from unittest import mock

import pytest
import torch
import torch.nn as nn

from stratum_amd import upload as U
from stratum_amd.upload import (FP16_ATTR, NF4_ATTR, FP16StagedPayload, NF4Payload, NF4Prefetch,
                                _load_payload_from_cache, _replace_param_data, _save_payload_to_cache,
                                estimate_module_upload_gib, ensure_prefetched_weights, free_weights,
                                prepare_fp16_staged, prepare_nf4, restore_module_buffers, snapshot_module_buffers)


def nf4_payload(shape=(2, 2), source_bytes=8, dtype=torch.float16):
    n = 1
    for s in shape:
        n *= s
    return NF4Payload(quantized=torch.zeros((n + 1) // 2, 1, dtype=torch.uint8),
                      absmax=torch.ones(max(1, -(-n // 64)), dtype=torch.float32),
                      code=torch.zeros(16, dtype=torch.float32), shape=tuple(shape), dtype=dtype, blocksize=64,
                      quant_type="nf4", source_numel=n, source_bytes=source_bytes, payload_bytes=36)


def no_pin(t):
    return t.detach().contiguous().cpu()


# ------------------------------------------------------ parameter replacement
@pytest.mark.parametrize("attr", [NF4_ATTR, FP16_ATTR])
def test_fallback_replacement_keeps_the_payload(attr):
    owner = nn.Module()
    p = nn.Parameter(torch.ones(2, 2, dtype=torch.float16), requires_grad=False)
    payload = nf4_payload() if attr == NF4_ATTR else FP16StagedPayload(torch.ones(2, 2), (2, 2), torch.float16, 8)
    setattr(p, attr, payload)
    owner.register_parameter("weight", p)
    with mock.patch.object(torch.nn.Parameter, "data", new_callable=mock.PropertyMock,
                           side_effect=RuntimeError("refused")):
        _replace_param_data(p, torch.empty(0, dtype=torch.float16), owner=owner, pname="weight")
    assert owner.weight is not p
    assert getattr(owner.weight, attr) is payload
    assert owner.weight.data.numel() == 0 and not owner.weight.requires_grad


def test_replacement_without_owner_is_a_silent_noop_when_refused():
    p = nn.Parameter(torch.ones(2), requires_grad=False)
    with mock.patch.object(torch.nn.Parameter, "data", new_callable=mock.PropertyMock,
                           side_effect=TypeError("refused")):
        _replace_param_data(p, torch.empty(0))


def test_estimate_counts_a_shared_payload_once():
    shared = nn.Parameter(torch.ones(2, 2), requires_grad=False)
    setattr(shared, NF4_ATTR, nf4_payload(source_bytes=8192))
    m = nn.Module()
    m.a = nn.Linear(2, 2, bias=False)
    m.b = nn.Linear(2, 2, bias=False)
    m.a.weight = shared
    m.b.weight = shared
    assert estimate_module_upload_gib(m) == 8192 / 10**9


# -------------------------------------------------------------- free / prefetch
def test_free_drops_only_staged_params():
    m = nn.Module()
    m.staged = nn.Linear(2, 2, bias=False).requires_grad_(False)
    m.plain = nn.Linear(2, 2, bias=False)
    setattr(m.staged.weight, NF4_ATTR, nf4_payload())
    assert free_weights(m) == 1
    assert m.staged.weight.numel() == 0 and m.plain.weight.numel() == 4
    assert free_weights(m) == 0  # already empty


def test_empty_prefetch_finalizes_without_a_gpu():
    assert NF4Prefetch([], torch.device("cuda:0")).finalize() == 0
    assert NF4Prefetch([], torch.device("cuda:0")).wait() == 0


def test_prefetched_ensure_chains_into_regular_ensure():
    m = nn.Linear(2, 2)
    with mock.patch.object(U, "ensure_weights", return_value=5) as ens:
        assert ensure_prefetched_weights(m, 0, NF4Prefetch([], torch.device("cuda:0"))) == 5
        ens.assert_called_once_with(m, 0)
        ens.reset_mock()
        assert ensure_prefetched_weights(m, 0, None) == 5
        ens.assert_called_once_with(m, 0)


def test_prefetch_device_mismatch_raises():
    with pytest.raises(ValueError):
        ensure_prefetched_weights(nn.Linear(2, 2), 1, NF4Prefetch([], torch.device("cuda:0")))


def test_prefetch_of_module_without_payloads_is_empty():
    assert U.prefetch_weights(nn.Linear(4, 4), 0).entries == []


# ------------------------------------------------------------------- cache v1
def _write_cache(tmp_path, **meta):
    path = tmp_path / "w.pt"
    torch.save({**meta, "quantized": torch.zeros(2, 1, dtype=torch.uint8), "absmax": torch.ones(1),
                "code": torch.zeros(16)}, path)
    return path


META = dict(version=1, shape=(2, 2), dtype="float16", blocksize=64, quant_type="nf4", source_numel=4,
            source_bytes=8)


def test_cache_accepts_exact_metadata(tmp_path):
    p = nn.Parameter(torch.ones(2, 2, dtype=torch.float16), requires_grad=False)
    with mock.patch.object(U, "_pin_cpu", side_effect=no_pin):
        pay = _load_payload_from_cache(_write_cache(tmp_path, **META), p, blocksize=64, quant_type="nf4")
    assert pay is not None and pay.blocksize == 64 and pay.quant_type == "nf4"
    assert pay.source_numel == 4 and pay.source_bytes == 8 and pay.shape == (2, 2) and pay.dtype == torch.float16


@pytest.mark.parametrize("key,value", [("blocksize", 128), ("version", 2), ("dtype", "bfloat16"),
                                       ("shape", (4, 1)), ("quant_type", "fp4"), ("source_bytes", 16)])
def test_cache_rejects_mismatched_metadata(tmp_path, key, value):
    p = nn.Parameter(torch.ones(2, 2, dtype=torch.float16), requires_grad=False)
    meta = dict(META)
    meta[key] = value
    assert _load_payload_from_cache(_write_cache(tmp_path, **meta), p, blocksize=64, quant_type="nf4") is None


def test_cache_rejects_unreadable_and_missing_files(tmp_path):
    p = nn.Parameter(torch.ones(2, 2, dtype=torch.float16), requires_grad=False)
    bad = tmp_path / "bad.pt"
    bad.write_bytes(b"not a torch file")
    assert _load_payload_from_cache(bad, p, blocksize=64, quant_type="nf4") is None
    assert _load_payload_from_cache(tmp_path / "missing.pt", p, blocksize=64, quant_type="nf4") is None


def test_cache_file_name_and_atomic_write(tmp_path):
    path = U._cache_path(tmp_path, "model.layers.0.mlp.module.gate_proj.weight")
    assert path.parent == tmp_path and path.suffix == ".pt"
    assert path.name.endswith("model.layers.0.mlp.gate_proj.weight.pt")  # wrapper ".module." removed
    assert len(path.name.split("-", 1)[0]) == 12
    pay = nf4_payload()
    _save_payload_to_cache(path, pay)
    assert path.exists() and not path.with_name(path.name + ".tmp").exists()
    obj = torch.load(path, weights_only=True)
    assert obj["version"] == 1 and obj["shape"] == (2, 2) and obj["dtype"] == "float16"


# ------------------------------------------------------------- FP16-staged path
def fp16_module():
    m = nn.Module()
    m.big = nn.Linear(64, 64, bias=False).requires_grad_(False)
    m.small = nn.Linear(2, 2, bias=False).requires_grad_(False)
    m.train_me = nn.Linear(64, 64, bias=False)
    return m


def test_fp16_staging_scope_and_idempotence():
    m = fp16_module()
    with mock.patch.object(U, "_pin_cpu", side_effect=no_pin):
        assert prepare_fp16_staged(m, min_numel=64, verbose=False) == 1
        assert prepare_fp16_staged(m, min_numel=64, verbose=False) == 0
    pay = getattr(m.big.weight, FP16_ATTR)
    assert isinstance(pay, FP16StagedPayload) and pay.shape == (64, 64)
    assert pay.source_bytes == 64 * 64 * m.big.weight.dtype.itemsize
    assert m.big.weight.numel() == 0
    assert not hasattr(m.small.weight, FP16_ATTR) and not hasattr(m.train_me.weight, FP16_ATTR)


def test_free_keeps_the_host_copy_of_fp16_staged():
    m = nn.Linear(8, 8, bias=False).requires_grad_(False)
    with mock.patch.object(U, "_pin_cpu", side_effect=no_pin):
        prepare_fp16_staged(m, min_numel=8, verbose=False)
    pay = getattr(m.weight, FP16_ATTR)
    m.weight.data = pay.data.clone()
    assert free_weights(m) == 1 and m.weight.numel() == 0 and pay.data.numel() == 64


# ------------------------------------------------- prepare_nf4 (quantizer stubbed)
class _Recorder:
    """Stand-in for the GPU quantizer: records the 2-D shape it receives."""

    def __init__(self):
        self.shapes = []

    def __call__(self, weight, blocksize, compress_statistics, quant_type, rounding="argmin"):
        from stratum_amd.functional import QuantState
        self.shapes.append(tuple(weight.shape))
        n = weight.numel()
        state = QuantState(absmax=torch.zeros(-(-n // blocksize)), shape=weight.shape, code=torch.zeros(16),
                           blocksize=blocksize, quant_type=quant_type, dtype=weight.dtype)
        return torch.zeros((n + 1) // 2, 1, dtype=torch.uint8), state


def run_prepare(module, **kw):
    rec = _Recorder()
    with mock.patch.object(U, "_pin_cpu", side_effect=no_pin), mock.patch.object(U, "quantize_4bit", rec):
        stats = prepare_nf4(module, verbose=False, **kw)
    return stats, rec.shapes


def test_prepare_nf4_stages_2d_weight():
    m = nn.Module()
    m.register_parameter("weight", nn.Parameter(torch.randn(8, 8, dtype=torch.float16), requires_grad=False))
    stats, shapes = run_prepare(m, min_numel=8)
    assert stats.tensors == 1 and (8, 8) in shapes
    pay = getattr(m.weight, NF4_ATTR)
    assert pay.shape == (8, 8) and pay.dtype == torch.float16 and m.weight.numel() == 0


def test_prepare_nf4_flattens_stacked_experts_but_keeps_3d_shape():
    m = nn.Module()
    m.register_parameter("gate_up_proj", nn.Parameter(torch.randn(4, 16, 8, dtype=torch.float16),
                                                       requires_grad=False))
    stats, shapes = run_prepare(m, min_numel=8)
    assert (64, 8) in shapes
    assert getattr(m.gate_up_proj, NF4_ATTR).shape == (4, 16, 8)
    assert stats.source_bytes == 4 * 16 * 8 * 2


def test_prepare_nf4_skips_trainable_1d_small_and_integer_params():
    m = nn.Module()
    m.register_parameter("trainable", nn.Parameter(torch.randn(8, 8, dtype=torch.float16)))
    m.register_parameter("bias", nn.Parameter(torch.randn(64, dtype=torch.float16), requires_grad=False))
    m.register_parameter("tiny", nn.Parameter(torch.randn(2, 2, dtype=torch.float16), requires_grad=False))
    m.register_parameter("ids", nn.Parameter(torch.zeros(8, 8, dtype=torch.int32), requires_grad=False))
    stats, shapes = run_prepare(m, min_numel=8)
    assert stats.tensors == 0 and shapes == []


def test_prepare_nf4_counts_an_existing_payload_without_requantizing():
    m = nn.Module()
    m.register_parameter("weight", nn.Parameter(torch.empty(0, dtype=torch.float16), requires_grad=False))
    m.weight.data = torch.empty(8, 8, dtype=torch.float16)
    setattr(m.weight, NF4_ATTR, nf4_payload((8, 8), source_bytes=128))
    stats, shapes = run_prepare(m, min_numel=8)
    assert stats.tensors == 1 and stats.source_bytes == 128 and shapes == []


def test_prepare_nf4_cache_miss_writes_then_hits(tmp_path):
    def mod():
        m = nn.Module()
        m.register_parameter("weight", nn.Parameter(torch.randn(8, 8, dtype=torch.float16), requires_grad=False))
        return m
    s1, shapes1 = run_prepare(mod(), min_numel=8, cache_dir=tmp_path)
    assert (s1.cache_misses, s1.cache_writes, s1.cache_hits) == (1, 1, 0) and shapes1
    s2, shapes2 = run_prepare(mod(), min_numel=8, cache_dir=tmp_path)
    assert (s2.cache_misses, s2.cache_writes, s2.cache_hits) == (0, 0, 1) and shapes2 == []


def test_prepare_nf4_from_cache_returns_none_on_first_miss(tmp_path):
    m = nn.Module()
    m.register_parameter("weight", nn.Parameter(torch.randn(8, 8, dtype=torch.float16), requires_grad=False))
    assert U.prepare_nf4_from_cache(m, tmp_path, min_numel=8, verbose=False) is None
    assert U.prepare_nf4_from_cache(m, None) is None


def test_compression_ratio():
    s = U.NF4Stats(source_bytes=200, payload_bytes=50)
    assert s.compression == 4.0 and U.NF4Stats().compression == 0.0


# ------------------------------------------------------ buffer snapshot/restore
def bufs():
    m = nn.Module()
    m.register_buffer("mean", torch.zeros(4))
    m.register_buffer("var", torch.ones(4))
    m.register_buffer("empty", torch.empty(0))
    inner = nn.Module()
    inner.register_buffer("stats", torch.zeros(2))
    m.add_module("sub", inner)
    return m


def test_snapshot_is_a_clone_of_nonempty_buffers():
    m = bufs()
    snap = snapshot_module_buffers(m)
    assert set(snap) == {"mean", "var", "sub.stats"}
    m.mean.fill_(9)
    assert torch.all(snap["mean"] == 0)


def test_restore_reverts_mutations_and_empty_snapshot_is_noop():
    m = bufs()
    snap = snapshot_module_buffers(m)
    m.mean.fill_(5)
    m.sub.stats.fill_(3)
    assert restore_module_buffers(m, snap) == 3
    assert torch.all(m.mean == 0) and torch.all(m.sub.stats == 0)
    m.var.fill_(7)
    assert restore_module_buffers(m, {}) == 0 and torch.all(m.var == 7)
    assert snapshot_module_buffers(nn.Linear(2, 2)) == {}


def test_public_names_mirror_the_reference_exports():
    import stratum_amd
    for name in ("prepare_nf4", "prepare_nf4_from_cache", "prepare_fp16_staged", "upload_stream", "NF4Stats",
                 "estimate_module_upload_gib", "NF4Prefetch", "ensure_prefetched_weights", "prefetch_weights",
                 "FP16_ATTR", "FP16StagedPayload", "NF4Linear", "ensure_weights", "free_weights", "NF4_ATTR",
                 "NF4Payload", "snapshot_module_buffers", "restore_module_buffers"):
        assert hasattr(stratum_amd, name), name
    assert NF4_ATTR == "roundpipe_nf4_payload" and FP16_ATTR == "stratum_fp16_staged"
    assert isinstance(Path, type)


def test_nf4_linear_shape_metadata_without_gpu():
    from stratum_amd.functional import QuantState
    from stratum_amd.nf4_linear import NF4Linear
    st = QuantState(absmax=torch.ones(4), shape=(16, 32), blocksize=64, quant_type="nf4", dtype=torch.float16)
    lin = NF4Linear(torch.zeros(256, 1, dtype=torch.uint8), st, bias=torch.zeros(16, dtype=torch.float16))
    assert lin.in_features == 32 and lin.out_features == 16 and not lin.bias.requires_grad
