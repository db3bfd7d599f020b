"""Arena planning from a checkpoint's headers (CPU: no pinned memory involved).

plan_arena_bytes reads only the safetensors headers of a local checkpoint and
must give exactly the packed INT4 bytes the loader will register: n rows of
ceil(k/8) words per matrix, k padded to the group size when asked, and the
transposed shape for the down_proj_T registration.
"""
import json

import torch


def _checkpoint(path, shapes, shards=2):
    from safetensors.torch import save_file

    parts, wm = [{} for _ in range(shards)], {}
    for i, (name, shape) in enumerate(shapes.items()):
        parts[i % shards][name] = torch.zeros(*shape, dtype=torch.bfloat16)
        wm[name] = f"s{i % shards}.safetensors"
    for s in range(shards):
        save_file(parts[s], str(path / f"s{s}.safetensors"))
    (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))


def test_plan_arena_bytes_from_headers(tmp_path):
    from soinfer.offload import load_hf_checkpoint as ld

    H, I = 200, 264
    sh = {"self_attn.q_proj.weight": (256, H), "self_attn.k_proj.weight": (128, H),
          "self_attn.v_proj.weight": (128, H), "self_attn.o_proj.weight": (H, 256),
          "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H), "mlp.down_proj.weight": (H, I)}
    _checkpoint(tmp_path, {f"model.layers.{l}.{s}": v for l in range(3) for s, v in sh.items()})

    def words(k):
        return (k + 7) // 8 * 4

    unpadded = 3 * sum(n * words(k) for n, k in sh.values())
    assert ld.plan_arena_bytes(str(tmp_path), 3) == unpadded
    pad = lambda k: -(-k // 128) * 128  # noqa: E731
    padded = 3 * sum(n * words(pad(k)) for n, k in sh.values())
    assert ld.plan_arena_bytes(str(tmp_path), 3, group_size=128) == padded > unpadded
    down_T = ld.plan_arena_bytes(str(tmp_path), 3, suffixes=("mlp.down_proj.weight",), transpose=True,
                                 group_size=128)
    assert down_T == 3 * I * words(pad(H))
    assert ld.plan_arena_bytes(str(tmp_path), 2, suffixes=("mlp.up_proj.weight",)) == 2 * I * words(H)
    assert ld.packed_int4_bytes(17, 9) == 17 * 8
