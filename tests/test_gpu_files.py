"""Weights from files into HBM, through the C ABI.

GGUF: a model written to a file under llama.cpp's tensor names and read back
with Model.from_gguf holds exactly the same bytes in every tensor and decodes
to bit-identical logits.  .spm: each stream of a Granite expert layer emitted
as spm-granite-moe's layout.rs does lands on the device as exactly the GGUF
blocks (or the row-major router) it came from, and drives the expert FFN.
Both bars are exact: file placement moves bytes.
"""
import numpy as np
import pytest

import oracle
from emufpga_amd import _lib, spm
from emufpga_amd.gguf import GgufFile
from emufpga_amd.serve import DenseConfig, Model, Session
from tests import ggufw, npref

pytestmark = pytest.mark.gpu

SMALL_QWEN3 = DenseConfig(hidden=512, heads=4, kv_heads=2, head_dim=128, ffn=1024, vocab=1000, layers=2,
                          rope_theta=1e6, eps=1e-6, style=_lib.EMU_STYLE_QWEN3, encoding=_lib.Q6_K, tied=False,
                          qk_norm=True)
SMALL_SMOL = DenseConfig(hidden=576, heads=9, kv_heads=3, head_dim=64, ffn=1536, vocab=2048, layers=2,
                         rope_theta=1e5, eps=1e-5, style=_lib.EMU_STYLE_SMOL, encoding=_lib.Q8_0, tied=True,
                         qk_norm=False)
SMALL_GRANITE = DenseConfig(hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=0, vocab=300, layers=2,
                            rope_theta=1.5e6, eps=1e-6, style=_lib.EMU_STYLE_GRANITE, encoding=_lib.Q6_K, tied=True,
                            qk_norm=False, n_experts=8, experts_used=2, expert_ff=256, expert_encoding=_lib.Q6_K,
                            embed_scale=12.0, residual_scale=0.22, logit_div=6.0, score_mul=0.015625)


def f32_round(cfg: DenseConfig) -> DenseConfig:
    """The configuration as f32 metadata carries it."""
    d = dict(cfg.__dict__)
    for k in ("rope_theta", "eps", "embed_scale", "residual_scale", "logit_div", "score_mul"):
        d[k] = float(np.float32(d[k]))
    return DenseConfig(**d)


def write_model(tmp_path, model, name="m.gguf", mutate=None):
    meta, tensors = ggufw.model_file_tensors(model.cfg, model.host_weights())
    if mutate:
        tensors = mutate(tensors)
    p = tmp_path / name
    p.write_bytes(ggufw.gguf_bytes(meta, tensors, align=64))
    return p, tensors


@pytest.mark.parametrize("cfg", [SMALL_QWEN3, SMALL_SMOL, SMALL_GRANITE], ids=["qwen3", "smol", "granite"])
def test_gguf_model_holds_the_same_bytes_and_decodes_identically(ctx, tmp_path, cfg):
    a = Model(ctx, cfg)
    a.synth(31)
    p, tensors = write_model(tmp_path, a)
    b = Model.from_gguf(ctx, p)
    assert b.cfg == f32_round(cfg)
    _, back = ggufw.model_file_tensors(b.cfg, b.host_weights())
    assert [(n, d, t) for n, d, t, _ in back] == [(n, d, t) for n, d, t, _ in tensors]
    for (n, _, _, x), (_, _, _, y) in zip(tensors, back):
        assert bytes(x) == bytes(y), n
    prompts = np.array([[3, 1, 4, 1], [2, 7, 1, 8]], np.uint32)
    sa, sb = Session(a, 2, 48), Session(b, 2, 48)
    for t in range(4):
        na, la = sa.decode_step(prompts[:, t], want_logits=True)
        nb, lb = sb.decode_step(prompts[:, t], want_logits=True)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)) and np.array_equal(na, nb)
    assert np.array_equal(sa.generate(prompts, 12), sb.generate(prompts, 12))
    for m in (sa, sb, a, b):
        m.close()


def test_gguf_mismatches_are_refused_by_name(ctx, tmp_path):
    a = Model(ctx, SMALL_QWEN3)
    a.synth(2)

    def drop(ts):
        return [t for t in ts if t[0] != "blk.1.ffn_up.weight"]

    def retype(ts):  # the same matrix as Q8_0 blocks
        return [(n, d, 8, bytes(d[0] * d[1] // 32 * 34)) if n == "blk.0.attn_k.weight" else (n, d, t, x)
                for n, d, t, x in ts]

    def reshape(ts):  # 256 rows of 512 declared as 512 rows of 256: same bytes, wrong shape
        return [(n, (d[1], d[0]) if n == "blk.1.attn_v.weight" else d, t, x) for n, d, t, x in ts]

    cases = [(drop, "missing tensor blk.1.ffn_up.weight"), (retype, "tensor blk.0.attn_k.weight: dtype 8"),
             (reshape, "tensor blk.1.attn_v.weight: dtype 14, 2 dims [256, 512")]
    for i, (mutate, message) in enumerate(cases):
        p, _ = write_model(tmp_path, a, f"bad{i}.gguf", mutate)
        b = Model(ctx, SMALL_QWEN3)
        with GgufFile(p) as f:
            with pytest.raises(_lib.EmuError) as e:
                b.load_gguf(f)
        assert message in str(e.value), str(e.value)
        b.close()
    a.close()


def test_large_range_upload_crosses_the_staging_buffers(ctx, tmp_path):
    n = (150 << 20) + 12344  # several 64 MiB chunks and a ragged tail
    data = np.random.default_rng(9).integers(0, 256, n, dtype=np.uint8).tobytes()
    p = tmp_path / "big.gguf"
    p.write_bytes(ggufw.gguf_bytes([], [("blob", (n // 4,), 0, data)]))
    with GgufFile(p) as f:
        buf = ctx.alloc(n)
        f.upload(ctx, "blob", buf.addr, relative_offset=3, length=n - 10)
        got = buf.read(np.uint8, n - 10)
        assert got.tobytes() == data[3:n - 7]
        with pytest.raises(Exception, match="requested range exceeds tensor blob"):
            f.upload(ctx, "blob", buf.addr, relative_offset=8, length=n - 4)
        buf.free()


def granite_layer_file(tmp_path, rng, E=8, W=512, FF=256):
    gate = npref.random_blocks(_lib.Q6_K, E * FF * W // 256, rng)
    up = npref.random_blocks(_lib.Q6_K, E * FF * W // 256, rng)
    down = npref.random_blocks(_lib.Q6_K, E * W * FF // 256, rng)
    router = rng.normal(size=(E, W)).astype(np.float32)
    tensors = [("blk.0.ffn_gate_inp.weight", (W, E), 0, router.tobytes()),
               ("blk.0.ffn_gate_exps.weight", (W, FF, E), 14, gate.tobytes()),
               ("blk.0.ffn_up_exps.weight", (W, FF, E), 14, up.tobytes()),
               ("blk.0.ffn_down_exps.weight", (FF, W, E), 14, down.tobytes())]
    p = tmp_path / "layer.gguf"
    p.write_bytes(ggufw.gguf_bytes([], tensors))
    return p, router, gate, up, down


def test_spm_expert_layer_streams_land_as_their_gguf_blocks(ctx, tmp_path):
    E, W, FF = 8, 512, 256
    rng = np.random.default_rng(41)
    p, router, gate, up, down = granite_layer_file(tmp_path, rng, E, W, FF)
    experts = [1, 5, 6]
    with GgufFile(p) as f:
        data = spm.emit_moe_layer(f, 0, experts, E, W, FF)
    r = spm.SpmReader(data)
    assert len(r.descriptors) == 1 + 3 * len(experts)
    assert r.descriptors[1] == spm.OpDescriptor(FF, W, 256, spm.Encoding.Q6K, 1)
    # 214-byte groups: an inert 1.0 scale then one 210-byte block
    assert len(data) == 32 + 32 * 10 + W * (4 + 4 * E) + len(experts) * 3 * (FF * W // 256) * 214
    rb = spm.device_bytes(r.descriptors[0])
    d_router = ctx.alloc(rb)
    assert r.upload_stream(ctx, d_router.addr, rb) == 0
    assert np.array_equal(d_router.read(np.float32).reshape(E, W).view(np.uint32), router.view(np.uint32))
    per_up, per_down = FF * (W // 256) * 210, W * (FF // 256) * 210
    placed = {}
    for e in experts:
        for name, src, size in (("up", up, per_up), ("gate", gate, per_up), ("down", down, per_down)):
            buf = ctx.alloc(size)
            r.upload_stream(ctx, buf.addr, size)
            got = buf.read(np.uint8)
            assert np.array_equal(got, src.reshape(-1)[e * size:(e + 1) * size]), (e, name)
            placed[(e, name)] = got
    assert r.next_group() is None
    # the placed expert blocks drive the selected-expert FFN (3 experts, compact ids)
    k, T = 2, 3
    g3 = np.concatenate([placed[(e, "gate")] for e in experts])
    u3 = np.concatenate([placed[(e, "up")] for e in experts])
    d3 = np.concatenate([placed[(e, "down")] for e in experts])
    x = rng.normal(size=(T, W)).astype(np.float32)
    ids = np.array([[0, 2], [1, 2], [0, 1]], np.int64)
    wts = np.array([[0.6, 0.4], [0.5, 0.5], [0.3, 0.7]], np.float32)
    from tests.test_gpu_moe import run_gpu
    got = run_gpu(ctx, _lib.Q6_K, _lib.Q6_K, g3, u3, d3, None, 3, W, FF, k, _lib.EMU_ACT_SILU, x, ids, wts)
    ref = oracle.moe_ffn(_lib.Q6_K, _lib.Q6_K, g3, u3, d3, None, 3, W, FF, k, oracle.OR_ACT_SILU, x, ids, wts)
    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))


@pytest.mark.parametrize("enc,gs,rows,cols", [(spm.Encoding.Q8_0, 64, 3, 64), (spm.Encoding.Q5K, 512, 3, 256),
                                              (spm.Encoding.Q6K, 768, 5, 512), (spm.Encoding.F32, 7, 5, 3)])
def test_spm_streams_with_multi_block_and_short_groups(ctx, enc, gs, rows, cols):
    rng = np.random.default_rng(gs + rows)
    n = rows * cols
    if enc == spm.Encoding.F32:
        w = rng.normal(size=(rows, cols)).astype(np.float32)
        stream = w.T.reshape(-1).tobytes()  # column-major
        per, want = 4, w.tobytes()
    else:
        e = {spm.Encoding.Q8_0: _lib.Q8_0, spm.Encoding.Q5K: _lib.Q5_K, spm.Encoding.Q6K: _lib.Q6_K}[enc]
        be = npref.BLOCK_ELEMS[e]
        blocks = npref.random_blocks(e, n // be, rng).reshape(-1)
        stream, want, per = blocks.tobytes(), blocks.tobytes(), None
    d = spm.OpDescriptor(rows, cols, gs, enc)
    w_ = spm.SpmWriter([spm.OpDescriptor(1, 4, 4, spm.Encoding.TERNARY2_F32_I32), d])
    w_.write_raw_group(1.0, b"\x55", 4)
    at = 0
    for g in range(0, n, gs):
        cnt = min(gs, n - g)
        nb = enc.bytes_for(cnt)
        w_.write_raw_group(1.0, stream[at:at + nb], cnt)
        at += nb
    r = spm.SpmReader(w_.finish())
    buf = ctx.alloc(len(want))
    with pytest.raises(spm.FileError, match="no device layout for encoding profile 1"):
        r.upload_stream(ctx, buf.addr, len(want))
    r.next_group()
    with pytest.raises(spm.FileError, match="needs"):
        r.upload_stream(ctx, buf.addr, len(want) - 1)
    assert r.upload_stream(ctx, buf.addr, len(want)) == 1
    assert buf.read(np.uint8).tobytes() == want
    with pytest.raises(spm.FileError, match="no stream left"):
        r.upload_stream(ctx, buf.addr, len(want))
