"""GPU: GGUF tensors uploaded verbatim into HBM and the executor dispatch over them.

A checkpoint holding the decode path's tensor kinds (rank-2 Q4_K/Q6_K/Q8_0
matrices, an F32 router, stacked Q4_K/Q6_K expert tensors, a 1-D F32 norm)
is written to disk, parsed by pyrite_amd.gguf and uploaded by
ResidentTensors.  Checks:

- the HBM arena holds every tensor's file bytes exactly, with a staging buffer
  small enough that tensors straddle chunk boundaries;
- tensor_matvec / matrix_matvec / slice_matvec / grouped_matvec over the resident bytes equal
  the device matvec over separately uploaded copies bit for bit, and the
  oracle's fp64 matvec within 1e-4*||x||_2*max|row|;
- the expert slice's byte range is the oracle's (pyrite/qwen3_moe.py:364-398);
- matrix_rows is bit-exact against the oracle's dequantization;
- lm_head's ids are the oracle's first max; the MoE layer built from
  resident tensors routes to the oracle's experts;
- the reference executor's shape and range errors (pyrite/executor.py:481-594).
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import gguf_writer as gw
from tests.gpu_util import announce, assert_matvec_close

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

H, I, E, K = 512, 256, 8, 2


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory, orc):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pyrite_amd import _lib
    from pyrite_amd.gguf import GGUFReader
    _lib.load()
    rng = np.random.default_rng(7)

    def q(t, rows, cols, seed):
        return orc.quantize(t, orc.normal(seed, rows * cols, 0.0, 0.02)).astype(np.uint8)

    host = {
        "blk.0.attn_q.weight": ((H, 3 * 256), 12, q(12, 3 * 256, H, 1)),
        "blk.0.ffn_down.weight": ((3 * 256, H), 14, q(14, H, 3 * 256, 2)),
        "token_embd.weight": ((H, 40), 8, q(8, 40, H, 3)),
        "output.weight": ((H, 1000), 14, q(14, 1000, H, 4)),
        "blk.0.ffn_gate_inp.weight": ((H, E), 0, orc.normal(5, E * H, 0.0, 0.02).astype(np.float32).view(np.uint8)),
        "blk.0.ffn_gate_exps.weight": ((H, I, E), 12, q(12, E * I, H, 6)),
        "blk.0.ffn_up_exps.weight": ((H, I, E), 12, q(12, E * I, H, 7)),
        "blk.0.ffn_down_exps.weight": ((I, H, E), 14, q(14, E * H, I, 8)),
        "output_norm.weight": ((H,), 0, rng.standard_normal(H).astype(np.float32).view(np.uint8)),
    }
    w = gw.Writer()
    w.kv("qwen3moe.expert_count", gw.U32, E)
    # directory order differs from payload order
    names = list(host)
    offsets = {}
    off = 0
    for n in reversed(names):
        offsets[n] = off
        off = -(-(off + host[n][2].nbytes) // 32) * 32
    for n in names:
        dims, t, payload = host[n]
        w.tensor(n, dims, t, payload.tobytes(), offset=offsets[n])
    path = tmp_path_factory.mktemp("gguf") / "layer.gguf"
    path.write_bytes(w.bytes())
    return GGUFReader(path), host


@pytest.fixture(scope="module")
def res(ckpt):
    from pyrite_amd.resident import ResidentTensors
    reader, _ = ckpt
    return ResidentTensors(reader, staging_bytes=4096 + 68)  # chunks straddle every tensor boundary


def test_arena_holds_file_bytes(ckpt, res):
    reader, host = ckpt
    announce("resident", "arena bytes", f"{res.nbytes} B")
    for name, (_, _, payload) in host.items():
        assert res.view(name).data_ptr() % 256 == 0
        assert np.array_equal(res.view(name).cpu().numpy(), payload), name
        assert reader.read_tensor(reader.tensor(name)) == payload.tobytes()
    # a subset upload holds just those tensors
    from pyrite_amd.resident import ResidentTensors
    sub = ResidentTensors(reader, names=["output.weight"])
    assert sub.names() == ("output.weight",)
    assert np.array_equal(sub.view("output.weight").cpu().numpy(), host["output.weight"][2])


@pytest.mark.parametrize("name", ["blk.0.attn_q.weight", "blk.0.ffn_down.weight", "output.weight"])
@pytest.mark.parametrize("batch", [1, 8])
def test_tensor_and_row_range_matvec(orc, ckpt, res, name, batch):
    from pyrite_amd import device
    _, host = ckpt
    (cols, rows), t, payload = host[name]
    announce("resident", "matvec", name, f"{rows}x{cols}", f"batch={batch}")
    x = orc.normal(100 + batch, batch * cols).astype(np.float32).reshape(batch, cols)
    xd = torch.from_numpy(x).cuda()
    y = res.tensor_matvec(name, rows, cols, xd).cpu().numpy()
    same = device.matvec(t, torch.from_numpy(payload).cuda(), xd, rows, cols).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), same.view(np.uint32))
    deq = orc.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
    rmax = np.abs(deq).max(axis=1)
    for b in range(batch):
        ref = orc.matvec(t, payload, x[b].astype(np.float64), rows, cols)
        assert_matvec_close(y[b], ref, x[b], rmax, f"{name} b={b}")
    if batch == 1:
        first, count = rows // 3, rows // 2
        part = res.matrix_matvec(name, first, count, xd[0]).cpu().numpy()
        assert np.array_equal(part.view(np.uint32), y[0, first:first + count].view(np.uint32))
        assert res.matrix_matvec(name, rows, 0, xd[0]).numel() == 0


@pytest.mark.parametrize("batch", [1, 2, 8])
def test_grouped_matvec_equals_single_calls(orc, ckpt, res, batch):
    """The same Q4_K tensor twice in one grouped launch equals the single launch, bit for bit."""
    _, host = ckpt
    (cols, rows), _, _ = host["blk.0.attn_q.weight"]
    announce("resident", "grouped", f"batch={batch}")
    x = torch.from_numpy(orc.normal(500 + batch, batch * cols).astype(np.float32).reshape(batch, cols)).cuda()
    names = ["blk.0.attn_q.weight", "blk.0.ffn_gate_exps.weight"]
    with pytest.raises(ValueError, match="rank-2"):
        res.grouped_matvec(names, x)
    with pytest.raises(ValueError, match="one GGML type"):
        res.grouped_matvec(["blk.0.attn_q.weight", "output.weight"], x)
    ys = res.grouped_matvec(["blk.0.attn_q.weight", "blk.0.attn_q.weight"], x)
    single = res.tensor_matvec("blk.0.attn_q.weight", rows, cols, x).cpu().numpy()
    for y in ys:
        assert y.shape == (batch, rows)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), single.view(np.uint32))


@pytest.mark.parametrize("comp, rows, cols", [("gate", I, H), ("up", I, H), ("down", H, I)])
def test_expert_slice_matvec(orc, ckpt, res, comp, rows, cols):
    from pyrite_amd import device
    from pyrite_amd.ggml_types import spec
    _, host = ckpt
    name = f"blk.0.ffn_{comp}_exps.weight"
    _, t, payload = host[name]
    x = orc.normal(200, cols).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    b = spec(t)
    per = rows * cols // b.block_size * b.bytes_per_block
    for e in (0, 3, E - 1):
        announce("resident", "slice", name, f"expert={e}")
        s = res.expert_slice(name, e)
        assert (s.block_offset, s.byte_length, s.element_offset, s.element_count) == (e * per, per, e * rows * cols,
                                                                                      rows * cols)
        y = res.slice_matvec(name, e, rows, cols, xd).cpu().numpy()
        sl = payload[e * per:(e + 1) * per]
        same = device.matvec(t, torch.from_numpy(sl.copy()).cuda(), xd, rows, cols).cpu().numpy()
        assert np.array_equal(y.view(np.uint32), same.view(np.uint32))
        deq = orc.dequantize_rows(t, sl, rows, cols).reshape(rows, cols)
        assert_matvec_close(y, orc.matvec(t, sl, x.astype(np.float64), rows, cols), x, np.abs(deq).max(axis=1),
                            f"{name} e={e}")


def test_embedding_rows_are_exact(orc, ckpt, res):
    _, host = ckpt
    (cols, rows), t, payload = host["token_embd.weight"]
    announce("resident", "rows", "token_embd.weight")
    got = res.matrix_rows("token_embd.weight", 5, 7).cpu().numpy()
    ref = orc.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)[5:12]
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))
    got64 = res.matrix_rows("token_embd.weight", 0, rows, dtype=torch.float64).cpu().numpy()
    assert np.array_equal(got64.view(np.uint64), orc.dequantize_rows(t, payload, rows, cols).reshape(rows, cols)
                          .view(np.uint64))


def test_lm_head_ids(orc, ckpt, res):
    _, host = ckpt
    (cols, rows), t, payload = host["output.weight"]
    announce("resident", "lm_head", f"{rows}x{cols}")
    x = orc.rms_norm(orc.normal(300, 3 * cols).reshape(3, cols)[0]).astype(np.float32)
    xs = np.stack([x, -x, orc.normal(301, cols).astype(np.float32)])
    logits, ids = res.lm_head("output.weight", torch.from_numpy(xs).cuda())
    ids = ids.cpu().numpy()
    for b in range(3):
        ref = orc.matvec(t, payload, xs[b].astype(np.float64), rows, cols)
        assert ids[b] == orc.argmax_first(ref)


def test_moe_layer_from_resident_tensors(orc, ckpt, res):
    from pyrite_amd import device
    _, host = ckpt
    layer = res.moe_layer("blk.0.ffn_gate_inp.weight", "blk.0.ffn_gate_exps.weight", "blk.0.ffn_up_exps.weight",
                          "blk.0.ffn_down_exps.weight", k=K)
    assert (layer.n_experts, layer.hidden, layer.inter, layer.k) == (E, H, I, K)
    xs = orc.normal(400, 3 * H).astype(np.float32).reshape(3, H)
    announce("resident", "moe", f"E={E}", f"H={H}", f"I={I}", "batch=3")
    out, ids, _ = device.moe_ffn(layer, torch.from_numpy(xs).cuda())
    out, ids = out.cpu().numpy(), ids.cpu().numpy()
    r, g, u, d = (host[f"blk.0.ffn_{c}.weight"][2] for c in ("gate_inp", "gate_exps", "up_exps", "down_exps"))
    for b in range(3):
        ref, rids, _, _ = orc.moe_ffn(r, 0, g, 12, u, 12, d, 14, E, H, I, K, xs[b].astype(np.float64), True, 1.0)
        assert list(ids[b]) == list(rids)
        assert float(np.max(np.abs(out[b] - ref))) <= 1e-4 * float(np.max(np.abs(ref)))


def test_executor_errors(ckpt, res):
    x = torch.zeros(H, device="cuda")
    with pytest.raises(ValueError, match="expected GGML dimensions"):
        res.tensor_matvec("blk.0.attn_q.weight", H, 3 * 256, x)
    with pytest.raises(ValueError, match="shape mismatch"):
        res.matrix_matvec("blk.0.attn_q.weight", 0, 1, torch.zeros(H + 32, device="cuda"))
    with pytest.raises(ValueError, match="outside"):
        res.matrix_matvec("blk.0.attn_q.weight", 700, 100, x)
    with pytest.raises(ValueError, match="rank-2"):
        res.matrix_matvec("blk.0.ffn_gate_exps.weight", 0, 1, x)
    with pytest.raises(IndexError):
        res.expert_slice("blk.0.ffn_gate_exps.weight", E)
    with pytest.raises(ValueError, match="stacked 3D"):
        res.expert_slice("output.weight", 0)
    with pytest.raises(ValueError, match="shape mismatch"):
        res.slice_matvec("blk.0.ffn_gate_exps.weight", 0, I, H + 256, x)
    with pytest.raises(KeyError):
        res.view("absent.weight")
