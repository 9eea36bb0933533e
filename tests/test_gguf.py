"""The GGUF reader (qmatmul_gguf_*): metadata of every GGUF value type, tensor table and data views, alignment,
rejection of truncated and malformed files, and a GPU round trip GGUF -> qmatmul_prepare_weight -> GEMV."""
import os

import numpy as np
import pytest

import oracle
from arcinfer_amd import formats as F
from tests import gguf_writer as gw


def _sample(tmp_path, alignment=32):
    W1 = F.synth_weight(F.IQ4_XS, 64, 512, seed=1)       # [rows][bytes]
    W2 = F.synth_weight(F.Q8_0, 6 * 32, 256, seed=2)      # stacked "experts": dims [256, 32, 6]
    v = np.arange(10, dtype=np.float32)
    kvs = [("general.architecture", gw.STR, "qwen35"), ("general.alignment", gw.U32, alignment),
           ("x.u8", gw.U8, 200), ("x.i8", gw.I8, -5), ("x.u16", gw.U16, 60000), ("x.i16", gw.I16, -30000),
           ("x.u32", gw.U32, 4000000000), ("x.i32", gw.I32, -2000000000), ("x.f32", gw.F32, 0.5),
           ("x.bool", gw.BOOL, True), ("x.u64", gw.U64, 2 ** 40), ("x.i64", gw.I64, -(2 ** 40)), ("x.f64", gw.F64, 1e-6),
           ("tokenizer.tokens", gw.ARR, ["a", "bb", "ccc"], gw.STR), ("x.arr", gw.ARR, [1, 2, 3], gw.I32)]
    tens = [("blk.0.ffn_gate.weight", F.IQ4_XS, [512, 64], W1.tobytes()),
            ("blk.0.ffn_down_exps.weight", F.Q8_0, [256, 32, 6], W2.tobytes()),
            ("output_norm.weight", 0, [10], v.tobytes())]
    p = os.path.join(str(tmp_path), "m.gguf")
    gw.write_gguf(p, kvs, tens, alignment=alignment)
    return p, W1, W2, v


@pytest.mark.parametrize("alignment", [32, 64])
def test_gguf_metadata_and_tensors(qm, tmp_path, alignment):
    p, W1, W2, v = _sample(tmp_path, alignment)
    with qm.GgufFile(p) as g:
        assert len(g) == 3
        assert g.get_str("general.architecture") == "qwen35"
        assert g.get_int("x.u8") == 200 and g.get_int("x.i8") == -5 and g.get_int("x.u16") == 60000
        assert g.get_int("x.i16") == -30000 and g.get_int("x.u32") == 4000000000 and g.get_int("x.i32") == -2000000000
        assert g.get_float("x.f32") == 0.5 and g.get_int("x.bool") == 1 and g.get_int("x.u64") == 2 ** 40
        assert g.get_int("x.i64") == -(2 ** 40) and g.get_float("x.f64") == 1e-6
        with pytest.raises(qm.QMatmulError):
            g.get_int("general.architecture")
        with pytest.raises(qm.QMatmulError):
            g.get_int("no.such.key")
        t = g.tensor("blk.0.ffn_gate.weight")
        assert (t.qtype, t.dims, t.K, t.rows, t.nbytes) == (F.IQ4_XS, [512, 64], 512, 64, W1.nbytes)
        assert t.data % alignment == 0 and np.array_equal(t.numpy(), W1.ravel())
        t = g.tensor("blk.0.ffn_down_exps.weight")
        assert (t.qtype, t.dims, t.rows) == (F.Q8_0, [256, 32, 6], 192) and np.array_equal(t.numpy(), W2.ravel())
        t = g.tensor(2)
        assert t.name == "output_norm.weight" and np.array_equal(t.numpy().view(np.float32), v)
        with pytest.raises(qm.QMatmulError):
            g.tensor("missing.weight")


def test_gguf_split_model(qm, tmp_path):
    """name-00001-of-0000N.gguf opened from part 1 indexes every part's tensors (src/gguf.h:170-187); a name already
    indexed keeps its first part's data; a later part opened alone has only its own tensors; a missing part fails."""
    W1 = F.synth_weight(F.IQ4_XS, 32, 256, seed=3)
    W2 = F.synth_weight(F.Q8_0, 16, 256, seed=4)
    W3 = F.synth_weight(F.IQ4_XS, 32, 256, seed=5)
    part = os.path.join(str(tmp_path), "model-{:05d}-of-00003.gguf")
    split = lambda k: [("split.no", gw.U16, k), ("split.count", gw.U16, 3)]
    gw.write_gguf(part.format(1), [("general.architecture", gw.STR, "qwen35")] + split(0),
                  [("a.weight", F.IQ4_XS, [256, 32], W1.tobytes())])
    gw.write_gguf(part.format(2), split(1), [("b.weight", F.Q8_0, [256, 16], W2.tobytes()),
                                             ("a.weight", F.IQ4_XS, [256, 32], W3.tobytes())])
    gw.write_gguf(part.format(3), split(2), [("c.weight", F.IQ4_XS, [256, 32], W3.tobytes())])
    with qm.GgufFile(part.format(1)) as g:
        assert len(g) == 3 and g.get_int("split.count") == 3
        assert np.array_equal(g.tensor("a.weight").numpy(), W1.ravel())
        assert np.array_equal(g.tensor("b.weight").numpy(), W2.ravel())
        assert np.array_equal(g.tensor("c.weight").numpy(), W3.ravel())
    with qm.GgufFile(part.format(2)) as g:
        assert len(g) == 2 and np.array_equal(g.tensor("a.weight").numpy(), W3.ravel())
    os.remove(part.format(3))
    with pytest.raises(qm.QMatmulError, match="split part 3"):
        qm.GgufFile(part.format(1))


def test_gguf_rejects_malformed_files(qm, tmp_path):
    p, *_ = _sample(tmp_path)
    data = open(p, "rb").read()
    bad = os.path.join(str(tmp_path), "bad.gguf")
    cases = [b"GGUX" + data[4:],                      # magic
             data[:4] + (9).to_bytes(4, "little") + data[8:],  # version
             data[:40],                               # truncated metadata
             data[:len(data) - 100],                  # tensor data cut short
             data[:8] + (2 ** 60).to_bytes(8, "little") + data[16:]]  # absurd tensor count
    for c in cases:
        open(bad, "wb").write(c)
        with pytest.raises(qm.QMatmulError):
            qm.GgufFile(bad)
    with pytest.raises(qm.QMatmulError):
        qm.GgufFile(os.path.join(str(tmp_path), "missing.gguf"))


@pytest.mark.gpu
def test_gguf_to_gemv(qm, dev, tmp_path):
    import torch
    p, W1, W2, v = _sample(tmp_path)
    x = np.random.default_rng(3).standard_normal((1, 512)).astype(np.float32)
    with qm.GgufFile(p) as g:
        t = g.tensor("blk.0.ffn_gate.weight")
        w = qm.QWeight(t.qtype, t.numpy(), t.rows, t.K)  # straight from the mapping (host source)
    aq, asc, absum = qm.quantize_act(torch.from_numpy(x).to(dev), M_stride=16)
    y = qm.gemv(w, aq, asc, absum)
    torch.cuda.synchronize()
    ref = oracle.blockdot(F.IQ4_XS, W1, 512, aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy(), M=1)
    assert np.max(np.abs(y.cpu().numpy() - ref)) <= 1e-4 * np.max(np.abs(ref))
    w.release()


def test_gguf_every_weight_type_sized_by_its_block(qm, tmp_path):
    """A tensor of each of the 17 weight types: the reader sizes it from ggml's block geometry (elements and bytes per
    block, Q2_0 the reference's 64 / 18) and hands back the bytes written."""
    tens, ws = [], {}
    for i, qtype in enumerate(sorted(F.TYPE_NAMES)):
        W = F.synth_weight(qtype, 3, 512, seed=90 + i)
        ws[qtype] = W
        tens.append((f"t.{F.TYPE_NAMES[qtype]}", qtype, [512, 3], W.tobytes()))
    p = os.path.join(str(tmp_path), "types.gguf")
    gw.write_gguf(p, [("general.architecture", gw.STR, "x")], tens)
    with qm.GgufFile(p) as g:
        assert len(g) == 17
        for qtype, W in ws.items():
            t = g.tensor(f"t.{F.TYPE_NAMES[qtype]}")
            assert (t.qtype, t.K, t.rows, t.nbytes) == (qtype, 512, 3, W.nbytes), F.TYPE_NAMES[qtype]
            assert t.nbytes == 3 * F.row_bytes(qtype, 512) and np.array_equal(t.numpy(), W.ravel())
