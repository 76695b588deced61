"""Host logic of the checkpoint reader and the question-batch planner (CPU)."""

from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import save_file

from tests._util import gen
from d3trt_amd import ShardedCheckpoint, plan_batches
from d3trt_amd.checkpoint import layer_names


def write_checkpoint(root, layers=2, hidden=256, q=256, kv=128, inter=256, index=True, seed=0):
    """A bf16 checkpoint with the linear-path tensors of `layers` layers in one shard per layer (plus an
    unrelated tensor), named as the reference's checkpoint names them. Returns {name: tensor}."""
    g = gen(seed)
    everything = {}
    shards = {}
    for i in range(layers):
        names = layer_names(i)
        t = {
            names["input_layernorm"]: 0.1 * torch.randn(hidden, generator=g),
            names["post_attention_layernorm"]: 0.1 * torch.randn(hidden, generator=g),
            names["q_proj"]: 0.02 * torch.randn(q, hidden, generator=g),
            names["k_proj"]: 0.02 * torch.randn(kv, hidden, generator=g),
            names["v_proj"]: 0.02 * torch.randn(kv, hidden, generator=g),
            names["o_proj"]: 0.02 * torch.randn(hidden, q, generator=g),
            names["gate_proj"]: 0.02 * torch.randn(inter, hidden, generator=g),
            names["up_proj"]: 0.02 * torch.randn(inter, hidden, generator=g),
            names["down_proj"]: 0.02 * torch.randn(hidden, inter, generator=g),
        }
        t = {k: v.to(torch.bfloat16) for k, v in t.items()}
        shards[f"model-{i + 1:05d}-of-{layers:05d}.safetensors"] = t
        everything.update(t)
    extra = {"language_model.norm.weight": torch.ones(hidden, dtype=torch.bfloat16)}
    first = next(iter(shards))
    shards[first] = {**shards[first], **extra}
    everything.update(extra)
    for name, t in shards.items():
        save_file(t, str(root / name))
    save_file({"weight": torch.zeros(4, hidden)}, str(root / "readout.safetensors"))
    if index:
        wm = {k: name for name, t in shards.items() for k in t}
        (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {"total_size": 1234},
                                                                        "weight_map": wm}))
    return everything


@pytest.mark.parametrize("index", [True, False])
def test_sharded_checkpoint_reads_only_what_is_asked(tmp_path, index):
    tensors = write_checkpoint(tmp_path, index=index)
    ck = ShardedCheckpoint(tmp_path)
    assert set(ck.keys()) == set(tensors)  # the readout file is not part of the map
    assert len(ck.shards) == 2
    names = list(layer_names(1).values())
    got = ck.get_many(names)
    assert set(got) == set(names)
    for n in names:
        assert torch.equal(got[n], tensors[n])
    with pytest.raises(KeyError, match="not in the checkpoint"):
        ck.get_many(["language_model.layers.7.mlp.down_proj.weight"])
    assert ck.total_bytes() == (1234 if index else sum((tmp_path / s).stat().st_size for s in ck.shards))


def test_empty_directory_is_an_error(tmp_path):
    with pytest.raises(FileNotFoundError):
        ShardedCheckpoint(tmp_path)


def test_plan_batches_sorts_packs_and_covers_every_block():
    lengths = [5, 0, 16, 1, 16, 3, 9, 0, 12]
    for bs in (1, 2, 4, 8, None):
        batches = plan_batches(lengths, bs, bucket=8)
        seen = [i for b in batches for i in b.blocks]
        assert sorted(seen) == list(range(len(lengths)))  # every block exactly once
        flat_lengths = [lengths[i] for i in seen]
        assert flat_lengths == sorted(lengths)  # length-sorted, as backends/trtllm.py:151 orders them
        for b in batches:
            assert len(b.blocks) <= (bs or len(lengths))
            assert b.offsets[0] == 0 and b.rows == b.offsets[-1]
            assert all(b.offsets[k + 1] - b.offsets[k] == lengths[i] for k, i in enumerate(b.blocks))
            assert b.run_rows % 8 == 0 and b.rows <= b.run_rows < b.rows + 8
    assert len(plan_batches(lengths, None)) == 1
    assert [b.blocks for b in plan_batches([3, 1, 2], 2)] == [[1, 2], [0]]
    # ties keep input order (a stable sort)
    assert plan_batches([2, 2, 2], 3)[0].blocks == [0, 1, 2]


def test_plan_batches_rejects_bad_arguments():
    with pytest.raises(ValueError):
        plan_batches([1, -1], 2)
    with pytest.raises(ValueError):
        plan_batches([1, 2], 0)
    with pytest.raises(ValueError):
        plan_batches([1, 2], 2, bucket=0)
