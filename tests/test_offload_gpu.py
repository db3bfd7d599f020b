"""Pinned weight arena, copy streams and checkpoint-to-arena loading on the GPU.

Counterpart of the reference's tests/test_offload.py (PinnedWeightStore and
StreamManager semantics), plus: rows read in place through the arena's device
mapping, a double-buffered prefetch pipeline whose consumer is a real GEMV
(the write-after-read fence), and stream_load_layers on a small synthetic
safetensors checkpoint checked byte for byte against the quantizer and packer.
"""
import json

import pytest
import torch

from helpers import assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def off(cuda):
    from soinfer.offload import load_hf_checkpoint, stream_manager, weight_store

    return weight_store, stream_manager, load_hf_checkpoint


def test_register_views_and_bookkeeping(off):
    ws, _, _ = off
    a = torch.randint(0, 256, (8, 16), dtype=torch.uint8)
    b = torch.randint(0, 256, (4, 64), dtype=torch.uint8, device="cuda")  # any device
    store = ws.PinnedWeightStore(ws.plan_bytes([tuple(a.shape), tuple(b.shape)]))
    ha, hb = store.register("a", a), store.register("b", b)
    assert store.arena.is_pinned()
    assert store.handle("a") is ha and (ha.num_rows, ha.row_nbytes, ha.offset) == (8, 16, 0)
    assert hb.offset == a.numel() and store.bytes_used == store.bytes_total == a.numel() + b.numel()
    assert torch.equal(store.matrix_view(ha), a) and torch.equal(store.matrix_view(hb), b.cpu())
    for r in (0, 3, 7):
        assert torch.equal(store.row_view(ha, r), a[r])
    rows = torch.tensor([2, 0, 7, 2])
    got = store.rows_view(ha, rows)
    assert torch.equal(got, a[rows]) and got.is_contiguous()


def test_register_and_row_view_rejections(off):
    ws, _, _ = off
    store = ws.PinnedWeightStore(64)
    h = store.register("w", torch.zeros(2, 16, dtype=torch.uint8))
    with pytest.raises(IndexError):
        store.row_view(h, 2)
    with pytest.raises(ValueError):
        store.register("w", torch.zeros(1, 16, dtype=torch.uint8))  # duplicate name
    with pytest.raises(ValueError):
        store.register("x", torch.zeros(3, 16, dtype=torch.uint8))  # 48 > 32 bytes left
    with pytest.raises(ValueError):
        store.register("y", torch.zeros(16, dtype=torch.uint8))  # not 2D
    with pytest.raises(ValueError):
        ws.PinnedWeightStore(0)


def test_device_address_reads_rows_in_place(off):
    """A device gather from store.device_address(handle) returns the registered rows byte for byte (the arena
    is read through its device mapping, at the matrix's offset)."""
    import soinfer._C as C

    ws, _, _ = off
    g = torch.Generator().manual_seed(3)
    a = torch.randint(0, 256, (100, 48), dtype=torch.uint8, generator=g)
    b = torch.randint(0, 256, (300, 1024), dtype=torch.uint8, generator=g)
    store = ws.PinnedWeightStore(ws.plan_bytes([(100, 48), (300, 1024)]))
    store.register("a", a)
    hb = store.register("b", b)
    idx = torch.tensor([299, 0, 17, 17, 150], dtype=torch.int32, device="cuda")
    cnt = torch.tensor([5], dtype=torch.int32, device="cuda")
    dst = torch.zeros(5, 1024, dtype=torch.uint8, device="cuda")
    C.gather_rows_device_counted(store.device_address(hb), 300, 1024, idx, cnt, dst)
    assert torch.equal(dst.cpu(), b[idx.long().cpu()])


def test_prefetch_wait_and_rejections(off):
    ws, sm_mod, _ = off
    data = torch.randint(0, 256, (32, 128), dtype=torch.uint8)
    store = ws.PinnedWeightStore(data.numel())
    h = store.register("W", data)
    sm = sm_mod.StreamManager(num_buffers=2)
    buf = torch.empty(32, 128, dtype=torch.uint8, device="cuda")
    sm.prefetch(0, buf, store.matrix_view(h))
    sm.wait(0)
    assert torch.equal(buf.cpu(), data)
    sm.synchronize(0)
    with pytest.raises(ValueError):
        sm.prefetch(1, buf, torch.zeros(32, 128, dtype=torch.uint8))  # pageable host memory
    with pytest.raises(ValueError):
        sm.prefetch(1, buf[:16], store.matrix_view(h))  # shape mismatch
    with pytest.raises(ValueError):
        sm_mod.StreamManager(0)


@pytest.mark.parametrize("num_buffers", [2, 3])
def test_double_buffered_gemv_pipeline_write_after_read(off, num_buffers):
    """Layers of INT4 weights streamed through num_buffers device buffers while a GEMV consumes each one:
    wait(cur) -> GEMV -> mark_read_done(cur) -> prefetch layer i+nb-1 into the buffer freed longest ago. Every
    layer's output equals the GEMV over the same weights resident in HBM, bit for bit (a prefetch overwriting a
    buffer its GEMV is still reading would show up here)."""
    import soinfer.ops as ops

    ws, sm_mod, _ = off
    N, K, L = 2048, 2048, 12
    g = torch.Generator().manual_seed(11)
    layers = [torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, generator=g) for _ in range(L)]
    scales = [(torch.rand(N, K // 128, generator=g) * 0.01).cuda() for _ in range(L)]
    x = torch.randn(K, generator=g).half().cuda()
    store = ws.PinnedWeightStore(ws.plan_bytes([(N, K // 2)] * L))
    hs = [store.register(f"layer{i}", w) for i, w in enumerate(layers)]
    sm = sm_mod.StreamManager(num_buffers)
    bufs = [torch.empty(N, K // 2, dtype=torch.uint8, device="cuda") for _ in range(num_buffers)]
    for i in range(min(num_buffers - 1, L)):
        sm.prefetch(i, bufs[i], store.matrix_view(hs[i]))
    outs = []
    for i in range(L):
        cur = i % num_buffers
        sm.wait(cur)
        outs.append(ops.gemv_w4a16_group_lop3(bufs[cur], scales[i], x, K, 128))
        sm.mark_read_done(cur)
        nxt = i + num_buffers - 1
        if nxt < L:
            sm.prefetch(nxt % num_buffers, bufs[nxt % num_buffers], store.matrix_view(hs[nxt]))
    torch.cuda.synchronize()
    for i in range(L):
        want = ops.gemv_w4a16_group_lop3(layers[i].cuda(), scales[i], x, K, 128)
        assert torch.equal(outs[i], want), f"layer {i}"


def _write_checkpoint(path, layers, H, I, QH, KVH, seed, shards=2):
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(seed)
    shapes = {"self_attn.q_proj.weight": (QH, H), "self_attn.k_proj.weight": (KVH, H),
              "self_attn.v_proj.weight": (KVH, H), "self_attn.o_proj.weight": (H, QH),
              "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H), "mlp.down_proj.weight": (H, I)}
    tensors, weight_map = [{} for _ in range(shards)], {}
    for l in range(layers):
        for suffix, shape in shapes.items():
            name = f"model.layers.{l}.{suffix}"
            s = (l + len(weight_map)) % shards
            tensors[s][name] = (torch.randn(*shape, generator=g) * 0.02).to(torch.bfloat16)
            weight_map[name] = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
    for s in range(shards):
        save_file(tensors[s], str(path / f"model-{s + 1:05d}-of-{shards:05d}.safetensors"))
    (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    merged = {}
    for t in tensors:
        merged.update(t)
    return merged


@pytest.mark.parametrize("H,I", [(256, 384), (200, 264)])
def test_stream_load_layers_arena_bytes_and_gemv(off, tmp_path, H, I):
    """Every registered matrix equals pack_int4(quantize(w)) of the checkpoint tensor (down_proj_T of the
    transpose), the arena is exactly full (K padded to the group size when it is not a multiple), scales are
    on the GPU, and a GEMV over a matrix fetched from the arena matches the binary64 oracle."""
    import soinfer.ops as ops
    from soinfer.quant import formats, pack

    _, _, ld = off
    src = _write_checkpoint(tmp_path, 2, H, I, 256, 128, seed=H + I)
    store, mats = ld.stream_load_layers(str(tmp_path), 2, group_size=128, log_every=0, include_down_proj_t=True)
    assert store.bytes_used == store.bytes_total
    assert len(mats) == 2 * 8
    order = [store.handle(n).offset for n in mats]
    assert order == sorted(order), "registration order is layer by layer, suffix by suffix"
    for name, m in mats.items():
        w = src[name.replace("down_proj_T", "down_proj")].float()
        if "down_proj_T" in name:
            w = w.t().contiguous()
        qt = formats.quantize(w, formats.QuantConfig(bits=4, granularity="group", group_size=128))
        packed, packed_k = pack.pack_int4(qt.qweight)
        assert torch.equal(store.matrix_view(m.handle), packed), name
        assert m.scale.is_cuda and torch.equal(m.scale.cpu(), qt.scale)
        assert (m.n, m.k, m.packed_k) == (w.shape[0], w.shape[1], packed_k)
    m = mats["model.layers.1.mlp.gate_proj.weight"]
    x = torch.randn(m.packed_k, generator=torch.Generator().manual_seed(2)).half()
    x[m.k:] = 0
    y = ops.gemv_w4a16_group_lop3(store.matrix_view(m.handle).cuda(), m.scale, x.cuda(), m.packed_k, 128)
    ref = O.gemv_w4_f64(store.matrix_view(m.handle).numpy(), m.scale.cpu().numpy(), x.numpy(), m.packed_k, 128)
    assert_close(y, ref, "loaded gate_proj")


@pytest.mark.parametrize("fused", [True, False])
def test_engine_runs_a_loaded_checkpoint_from_host_memory(off, tmp_path, fused):
    """stream_load_layers -> decoder_weights_from_arena -> DecodeEngine: with the packed weights left in the pinned
    arena (offload=True; dense, DIP with no cache, cache-aware DIP) the engine generates exactly the tokens and
    hidden state of the resident engine over device copies of the same arena bytes."""
    from soinfer.runtime import decoder as D

    _, _, ld = off
    cfg = D.DecoderConfig(hidden=256, layers=3, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
                          group_size=128, max_seq=64)
    _write_checkpoint(tmp_path, cfg.layers, cfg.hidden, cfg.intermediate, cfg.q_heads * cfg.head_dim,
                      cfg.kv_heads * cfg.head_dim, seed=77)
    store, mats = ld.stream_load_layers(str(tmp_path), cfg.layers, group_size=128, log_every=0,
                                        include_down_proj_t=True)
    g = torch.Generator(device="cuda").manual_seed(5)

    def vec(n, std=1.0, base=0.0):
        return (torch.randn(n, generator=g, device="cuda") * std + base).half()

    embed = vec(cfg.vocab * cfg.hidden).view(cfg.vocab, cfg.hidden)
    lm_head = vec(cfg.vocab * cfg.hidden, 0.05).view(cfg.vocab, cfg.hidden)
    norms = [{"input_layernorm": vec(cfg.hidden, 0.1, 1.0), "post_attention_layernorm": vec(cfg.hidden, 0.1, 1.0),
              "q_norm": vec(cfg.head_dim, 0.1, 1.0), "k_norm": vec(cfg.head_dim, 0.1, 1.0)} for _ in range(cfg.layers)]
    final = vec(cfg.hidden, 0.1, 1.0)
    w_dev = D.decoder_weights_from_arena(store, mats, cfg, embed, lm_head, final, norms, device="cuda")
    w_host = D.decoder_weights_from_arena(store, mats, cfg, embed, lm_head, final, norms)
    assert not w_host.layers[0].qkv_Wq.is_cuda and w_host.layers[0].qkv_Wq.is_pinned()
    prompt = torch.randint(0, cfg.vocab, (5,), generator=torch.Generator().manual_seed(9)).tolist()
    k = cfg.intermediate // 2
    hot = [list(range(0, cfg.intermediate, 3)) for _ in range(cfg.layers)]
    dense = D.DecodeEngine(w_dev, "dense", max_new_tokens=6, fused=fused)
    want_dense = dense.generate(prompt, 6)
    dip = D.DecodeEngine(w_dev, "dip", dip_k=k, max_new_tokens=6, fused=fused)
    want_dip = dip.generate(prompt, 6)
    for mode, kw, want, ref in (("dense", {}, want_dense, dense),
                                ("cached_dip", dict(dip_k=k, hot_channels=[[] for _ in range(cfg.layers)]), want_dip,
                                 dip),
                                ("cached_dip", dict(dip_k=k, hot_channels=hot), want_dip, dip)):
        eng = D.DecodeEngine(w_host, mode, max_new_tokens=6, fused=fused, offload=True, **kw)
        for use_graph in (False, True):
            assert eng.generate(prompt, 6, use_graph=use_graph) == want, f"{mode} {kw.keys()} graph={use_graph}"
            assert torch.equal(eng.x_final, ref.x_final)
    with pytest.raises(ValueError):
        D.DecodeEngine(w_host, "dense")  # resident modes need the weights on the device
