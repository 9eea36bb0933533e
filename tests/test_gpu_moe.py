"""GPU parity of the MoE path: routing (ids and counts exact, weights within 1e-6, as tests/test_route.cpp), the
device-side permutation (scan / scatter invariants), and the full expert FFN against the oracle."""
import numpy as np
import pytest

import oracle
from arcinfer_amd import formats as F

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("NE,NU,T", [(256, 6, 7), (256, 8, 4096), (64, 4, 33), (128, 8, 5), (1024, 8, 6), (300, 8, 3)])
def test_route_matches_oracle(qm, dev, NE, NU, T):
    import torch
    rng = np.random.default_rng(11 + T)
    lg = (rng.standard_normal((T, NE)) * 2).astype(np.float32)
    if T == 7:
        lg[3, [5, 9, 200]] = 10.0  # ties: lower expert first
    if T in (6, 3):
        lg[0, [130, 70, 250]] = 9.0  # ties across 64-expert slices, the lower slice at the higher lane
        lg[1, :] = -np.inf  # fewer finite logits than selections: the rest in expert order
        lg[1, [NE - 1, 77, 3]] = [1.0, 2.0, 0.5]
        lg[2, 40:] = -np.inf
    ids, wts, counts = qm.moe_route(to_dev(lg, dev), NU)
    torch.cuda.synchronize()
    rid, rw, rc = oracle.moe_route(lg, NU)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.array_equal(counts.cpu().numpy(), rc)
    assert np.max(np.abs(wts.cpu().numpy() - rw)) < 1e-6


def _moe_setup(qm, dev, NE, E, Fd, T, NU, qtype, seed, types=None, extra_logit=False):
    """types: (gate, up, down) types, or qtype for all three; extra_logit: a router column NE (shared-expert gate)."""
    import torch
    tg, tu, td = types if types is not None else (qtype, qtype, qtype)
    Wg = F.synth_weight(tg, NE * Fd, E, seed=seed, sigma=0.05)
    Wu = F.synth_weight(tu, NE * Fd, E, seed=seed + 1, sigma=0.05)
    Wd = F.synth_weight(td, NE * E, Fd, seed=seed + 2, sigma=0.05)
    x = F.synth_activations(T, E, seed=seed + 3)
    lg = F.zipf_router_logits(T, NE + (1 if extra_logit else 0), seed=seed + 4)
    xt = to_dev(x, dev)
    aq, asc, absum = qm.quantize_act(xt)
    g, u, d = (qm.QWeight(t, to_dev(W, dev), W.shape[0], K) for t, W, K in ((tg, Wg, E), (tu, Wu, E), (td, Wd, Fd)))
    ws = qm.moe_workspace(T, NE, NU, E, Fd, device=dev)
    out = torch.zeros((T, E), dtype=torch.float32, device=dev)
    return dict(Wg=Wg, Wu=Wu, Wd=Wd, lg=lg, aq=aq, asc=asc, g=g, u=u, d=d, ws=ws, out=out, lgt=to_dev(lg, dev))


def moe_check(qm, s, types, NE, E, Fd, T, NU, tokens=None, escale=None, sh=None, sh_gated=True):
    """The GPU MoE output against the oracle. Decode sizes (no slot tiles): end to end, 1e-4. Slot tiles: in two
    stages, since the tile kernels sum the gate / up block products in another f32 order than the oracle and h's
    requantization per 32 (moe.cl:251-282) can then round a value next to a tie the other way, which moves the
    output by a whole int8 step of h: (1) the quantized h of every (token, k) slot against the oracle's (values
    equal but for one-step differences at no more than 0.2 % of them, scales within 1e-5); (2) down + combine
    recomputed by the oracle from the GPU's own h, within 1e-4 of the GPU output."""
    tg, tu, td = types
    got = s["out"].cpu().numpy()
    aqn, ascn = s["aq"].cpu().numpy(), s["asc"].cpu().numpy()
    if T * NU <= 64:
        ref = oracle.moe_forward(tg, s["Wg"], tu, s["Wu"], td, s["Wd"], NE, E, Fd, s["lg"], NU, aqn, ascn,
                                 escale=escale, sh=sh, sh_gated=sh_gated)
        assert rel_err(got, ref) < 1e-4
        return
    L = qm.moe_ws_layout(T, NE, NU, E, Fd)
    ws = s["ws"].cpu().numpy()
    view = lambda off, n, dt: np.frombuffer(ws[off:off + n * np.dtype(dt).itemsize].tobytes(), dtype=dt)
    inv = view(L.inv, T * NU, np.int32)
    hq = view(L.hq, L.slots * Fd, np.int8).reshape(L.slots, Fd)
    hsc = view(L.hsc, (Fd // 32) * L.slots, np.float32).reshape(Fd // 32, L.slots)
    ids, wts, _ = oracle.moe_route(s["lg"], NU, NE=NE, escale=escale)
    toks = range(T) if tokens is None else tokens
    ref = np.zeros((len(toks), E), dtype=np.float32)
    nflip = ntot = 0
    for j, t in enumerate(toks):
        for k in range(NU):
            e, slot = ids[t, k], inv[t * NU + k]
            a1, s1 = aqn[t:t + 1], ascn[:, t:t + 1]
            g = oracle.blockdot(tg, s["Wg"][e * Fd:(e + 1) * Fd], E, a1, s1, None)[0]
            u = oracle.blockdot(tu, s["Wu"][e * Fd:(e + 1) * Fd], E, a1, s1, None)[0]
            with np.errstate(over="ignore"):  # (exp(-g) = inf for very negative g: silu -> -0, as expf gives)
                h = (u * (g / (np.float32(1) + np.exp(-g)))).astype(np.float32)
            rq, rs, _ = oracle.quantize_act(h[None, :])
            d = np.abs(hq[slot].astype(np.int32) - rq[0].astype(np.int32))
            assert d.max() <= 1
            nflip += int(np.sum(d)); ntot += Fd
            assert np.max(np.abs(hsc[:, slot] - rs[:, 0]) / np.maximum(np.abs(rs[:, 0]), 1e-30)) < 1e-5
            y = oracle.blockdot(td, s["Wd"][e * E:(e + 1) * E], Fd, hq[slot:slot + 1],
                                np.ascontiguousarray(hsc[:, slot:slot + 1]), None)[0]
            ref[j] += wts[t, k] * y
        if sh is not None:
            with np.errstate(over="ignore"):
                gt = np.float32(1) / (np.float32(1) + np.exp(-np.float32(s["lg"][t, NE]))) if sh_gated else np.float32(1)
            ref[j] += gt * sh[t]
    assert nflip <= 0.002 * ntot
    assert rel_err(got[list(toks)], ref) < 1e-4


def check_permutation(qm, s, NE, E, Fd, T, NU):
    """The tile path's routing state in the workspace: slots of each expert contiguous, a bijection onto (token, k);
    the scan's counts, first slots, tile starts and tile list."""
    L = qm.moe_ws_layout(T, NE, NU, E, Fd)
    ws = s["ws"].cpu().numpy()
    view = lambda off, n, dt: np.frombuffer(ws[off:off + n * np.dtype(dt).itemsize].tobytes(), dtype=dt)
    ids = view(L.ids, T * NU, np.int32)
    inv = view(L.inv, T * NU, np.int32)
    stok = view(L.stok, T * NU, np.int32)
    assert np.array_equal(np.sort(inv), np.arange(T * NU))
    assert np.array_equal(stok[inv], np.arange(T * NU) // NU)
    counts = np.bincount(ids, minlength=NE)
    offs = np.concatenate([[0], np.cumsum(counts)[:-1]])
    assert np.all((offs[ids] <= inv) & (inv < offs[ids] + counts[ids]))
    tiles = view(L.tiles, 1 + 3 * L.max_tiles, np.int32)
    ntl = (counts + L.tile_rows - 1) // L.tile_rows
    assert tiles[0] == int(np.sum(ntl + (ntl & 1)))
    # the scan's outputs: counts, first slots, tile starts and the whole tile list
    assert np.array_equal(view(L.counts, NE, np.int32), counts)
    assert np.array_equal(view(L.cursor, NE, np.int32), offs)
    nt = (counts + L.tile_rows - 1) // L.tile_rows
    npad = nt + (nt & 1)  # (each expert's tiles start at an even index: an odd count gets an empty entry)
    assert np.array_equal(view(L.tstart, NE + 1, np.int32), np.concatenate([[0], np.cumsum(npad)]))
    want = [(e, offs[e] + k * L.tile_rows, min(L.tile_rows, counts[e] - k * L.tile_rows)) if k < nt[e]
            else (e, offs[e] + counts[e] - 1, 0) for e in range(NE) for k in range(npad[e])]
    assert np.array_equal(tiles[1:1 + 3 * len(want)].reshape(-1, 3), np.array(want, dtype=np.int32).reshape(-1, 3))


@pytest.mark.parametrize("qtype,NE,E,Fd,T,NU", [(F.IQ4_XS, 16, 512, 256, 64, 4), (F.IQ3_S, 8, 256, 512, 40, 2),
                                                (F.Q8_0, 8, 256, 256, 9, 3), (F.IQ4_XS, 256, 2048, 512, 48, 8),
                                                (F.Q4_0, 8, 256, 256, 70, 2), (F.IQ4_NL, 16, 512, 256, 33, 4),
                                                (F.IQ2_XXS, 8, 512, 256, 40, 2), (F.IQ3_XXS, 16, 256, 512, 33, 4),
                                                (F.IQ4_XS, 16, 512, 768, 40, 4), (F.Q8_0, 8, 256, 1024, 40, 4),
                                                (F.IQ3_XXS, 8, 256, 1024, 30, 4)])
def test_moe_grouped_matches_oracle(qm, dev, qtype, NE, E, Fd, T, NU):
    import torch
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, qtype, seed=NE + T)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    moe_check(qm, s, (qtype,) * 3, NE, E, Fd, T, NU)
    if T * NU <= 64:
        return  # (decode sizes take the GEMV-shaped kernels: no slot permutation is built)
    check_permutation(qm, s, NE, E, Fd, T, NU)


def test_moe_routing_state_large_T(qm, dev):
    """T >= 2048: several tokens per routing wave, the scatter's work-groups following the routing work-groups, a
    ragged last group (T not a multiple of the group's tokens); outputs checked on a few tokens."""
    import torch
    NE, E, Fd, T, NU = 64, 256, 256, 4100, 6
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=11)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    check_permutation(qm, s, NE, E, Fd, T, NU)
    moe_check(qm, s, (F.IQ4_XS,) * 3, NE, E, Fd, T, NU, tokens=[0, 1, 2047, 2048, 4095, 4096, 4099])


def test_moe_routing_state_many_experts(qm, dev):
    """NE = 600 (not a power of two, above 512: three experts per thread in the scatter's expert scan), tile path."""
    import torch
    NE, E, Fd, T, NU = 600, 256, 256, 300, 4
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=13)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    check_permutation(qm, s, NE, E, Fd, T, NU)
    moe_check(qm, s, (F.IQ4_XS,) * 3, NE, E, Fd, T, NU, tokens=[0, 1, 150, 299])


def test_moe_accumulate_and_determinism(qm, dev):
    import torch
    NE, E, Fd, T, NU = 32, 256, 256, 100, 4
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=5)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    first = s["out"].clone()
    for _ in range(3):  # slot order changes between runs (atomics); every slot's math does not
        qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
        torch.cuda.synchronize()
        assert torch.equal(s["out"], first)
    base = torch.full_like(first, 0.5)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], base, s["ws"], accumulate=1)
    torch.cuda.synchronize()
    assert torch.equal(base, 0.5 + first)


def test_moe_baseline_config_token_sample(qm, dev):
    """BASELINE config 4 at full size (256 experts, E 2048, F 512, T 4096, top-8, Zipf 1.1 router): the GPU output
    of 24 tokens against the oracle run on those tokens alone (tokens are independent)."""
    import torch
    NE, E, Fd, T, NU = 256, 2048, 512, 4096, 8
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=4)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    pick = list(range(8)) + list(range(2000, 2008)) + list(range(T - 8, T))
    moe_check(qm, s, (F.IQ4_XS,) * 3, NE, E, Fd, T, NU, tokens=pick)


@pytest.mark.parametrize("qtype,NE,E,Fd,T,NU", [(F.IQ4_XS, 256, 2048, 512, 1, 8), (F.IQ4_XS, 256, 2048, 512, 8, 8),
                                                (F.IQ3_S, 16, 1024, 1024, 3, 4), (F.Q8_0, 8, 512, 2048, 2, 2),
                                                (F.Q4_0, 8, 512, 512, 4, 2), (F.IQ4_NL, 16, 512, 256, 2, 4),
                                                (F.IQ2_XXS, 16, 1024, 512, 3, 4), (F.IQ3_XXS, 8, 512, 1024, 2, 2),
                                                (F.IQ4_XS, 300, 256, 256, 2, 4)])
def test_moe_decode_sizes_match_oracle(qm, dev, qtype, NE, E, Fd, T, NU):
    """T * NU <= 64: the GEMV-shaped decode kernels (gate/up -> h -> down + combine in k order)."""
    import torch
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, qtype, seed=7 * T + NU)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    ref = oracle.moe_forward(qtype, s["Wg"], qtype, s["Wu"], qtype, s["Wd"], NE, E, Fd, s["lg"], NU,
                             s["aq"].cpu().numpy(), s["asc"].cpu().numpy())
    assert rel_err(s["out"].cpu().numpy(), ref) < 1e-4
    first = s["out"].clone()
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    assert torch.equal(s["out"], first)
    base = torch.full_like(first, -0.25)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], base, s["ws"], accumulate=1)
    torch.cuda.synchronize()
    assert torch.equal(base, -0.25 + first)


@pytest.mark.parametrize("T", [1, 3, 6])
def test_moe_decode_masked_logits(qm, dev, T):
    """Rows with fewer finite router logits than selections (masked experts): the routing inside the decode gate/up
    kernel (T <= 4) and the separate route launch (T > 4) both fill the selection with the lowest -inf experts, at
    weight 0, as the oracle's stable order."""
    import torch
    NE, E, Fd, NU = 64, 256, 256, 4
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=5 + T)
    lg = s["lg"].copy()
    lg[0, :] = -np.inf
    lg[0, [9, 40]] = [0.5, 1.5]
    lgt = to_dev(lg, dev)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, lgt, NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    ref = oracle.moe_forward(F.IQ4_XS, s["Wg"], F.IQ4_XS, s["Wu"], F.IQ4_XS, s["Wd"], NE, E, Fd, lg, NU,
                             s["aq"].cpu().numpy(), s["asc"].cpu().numpy())
    got = s["out"].cpu().numpy()
    assert np.all(np.isfinite(got))
    rows = [rel_err(got[t], ref[t]) for t in range(T)]
    ids, _, _ = qm.moe_route(lgt, NU)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), oracle.moe_route(lg, NU)[0])
    # (per token row: h's int8 requantization per 32 may round one value the other way where the GPU's f32 h and
    #  the oracle's differ in the last place, moving that row by up to ~1e-3)
    assert max(rows) < 2e-3, rows


@pytest.mark.parametrize("T", [1, 4])
def test_moe_decode_graph_replays(qm, dev, T):
    """The decode-size path (routing inside the gate/up launch, then down) captured in a HIP graph: every replay, with
    eager launches of the same call between replays, matches the eager result bit for bit."""
    import torch
    NE, E, Fd, NU = 64, 512, 256, 4
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=31 + T)
    stream = torch.cuda.Stream()
    out_g = torch.zeros_like(s["out"])
    with torch.cuda.stream(stream):
        qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], out_g, s["ws"])
    stream.synchronize()
    eager = out_g.clone()
    ref = oracle.moe_forward(F.IQ4_XS, s["Wg"], F.IQ4_XS, s["Wu"], F.IQ4_XS, s["Wd"], NE, E, Fd, s["lg"], NU,
                             s["aq"].cpu().numpy(), s["asc"].cpu().numpy())
    assert rel_err(eager.cpu().numpy(), ref) < 1e-4
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], out_g, s["ws"])
    for _ in range(4):
        out_g.fill_(-1.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager)
        other = torch.zeros_like(eager)
        qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], other, s["ws"])
        torch.cuda.synchronize()
        assert torch.equal(other, eager)


# Expert types of the reference's moe_rg beyond the per-32 ones (Q6_K: per-16 int8 scales; IQ2_XS / IQ2_S: per-16
# 4-bit scales) and gate / up / down of different types, at decode sizes (GEMV-shaped kernels; gate and up of
# different types as two launches) and prompt sizes (slot tiles; gate-only then up-with-SwiGLU launches), plus the
# decode kernels' wider configurations (hidden sizes 4096 and 5120: 32 lanes and 4 or 8 blocks per lane; expert width
# 4096 in the down kernel).
@pytest.mark.parametrize("types,NE,E,Fd,T,NU", [
    ((F.Q6_K, F.Q6_K, F.Q6_K), 8, 512, 256, 2, 4), ((F.Q6_K, F.Q6_K, F.Q6_K), 8, 512, 256, 40, 2),
    ((F.IQ2_XS,) * 3, 8, 512, 256, 3, 4), ((F.IQ2_XS,) * 3, 8, 256, 512, 40, 2),
    ((F.IQ2_S,) * 3, 16, 512, 256, 2, 4), ((F.IQ2_S,) * 3, 8, 256, 256, 33, 4),
    ((F.IQ3_S, F.IQ3_S, F.Q6_K), 16, 1024, 512, 1, 8), ((F.IQ3_S, F.IQ3_S, F.Q6_K), 16, 512, 512, 48, 4),
    ((F.IQ3_S, F.IQ4_XS, F.Q8_0), 8, 512, 256, 4, 4), ((F.IQ3_S, F.IQ4_XS, F.Q8_0), 8, 512, 256, 40, 2),
    ((F.Q6_K, F.IQ2_S, F.IQ4_XS), 8, 256, 512, 3, 2), ((F.Q6_K, F.IQ2_S, F.IQ4_XS), 8, 256, 512, 64, 2),
    ((F.IQ4_XS,) * 3, 32, 4096, 512, 1, 8), ((F.IQ4_XS,) * 3, 16, 5120, 256, 4, 4),
    ((F.IQ4_XS,) * 3, 8, 512, 4096, 2, 4), ((F.IQ4_XS, F.IQ4_XS, F.Q6_K), 8, 512, 4096, 2, 4),
    # Q3_K (per-16 scales) and the reference's Q2_0, alone and mixed (zero/engine_moe.h:297-300)
    ((F.Q3_K,) * 3, 8, 512, 256, 1, 8), ((F.Q3_K,) * 3, 8, 512, 512, 40, 4), ((F.Q2_0,) * 3, 8, 512, 256, 3, 4),
    ((F.Q2_0,) * 3, 16, 512, 512, 48, 4), ((F.Q2_0, F.Q2_0, F.Q3_K), 8, 256, 512, 2, 4),
    ((F.Q3_K, F.IQ4_XS, F.Q2_0), 8, 512, 256, 40, 2),
])
def test_moe_expert_types_and_mixes(qm, dev, types, NE, E, Fd, T, NU):
    import torch
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, None, seed=3 * NE + T, types=types)
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
    torch.cuda.synchronize()
    moe_check(qm, s, types, NE, E, Fd, T, NU)
    for w in (s["g"], s["u"], s["d"]):
        w.release()


@pytest.mark.parametrize("T,NU", [(2, 4), (40, 4)])  # decode sizes / prompt sizes
@pytest.mark.parametrize("shared", ["gated", "plain", None])
@pytest.mark.parametrize("escale", [False, True])
def test_moe_expert_scales_and_shared_expert(qm, dev, T, NU, shared, escale):
    """moe.cl's options: expert scales on the routing weights (-DESCALE) and the shared expert's output added with
    its sigmoid gate from the router's column NE (or ungated, -DSH_NOGATE), against the extended oracle."""
    import torch
    if shared is None and not escale:
        pytest.skip("the plain call: covered by the other tests")
    NE, E, Fd = 16, 512, 256
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=T + NU, extra_logit=True)
    rng = np.random.default_rng(T)
    esc = rng.uniform(0.5, 2.0, NE).astype(np.float32) if escale else None
    sh = rng.standard_normal((T, E)).astype(np.float32) if shared else None
    qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"],
                   escale=None if esc is None else to_dev(esc, dev), sh=None if sh is None else to_dev(sh, dev),
                   sh_gated=shared == "gated")
    torch.cuda.synchronize()
    moe_check(qm, s, (F.IQ4_XS,) * 3, NE, E, Fd, T, NU, escale=esc, sh=sh, sh_gated=shared == "gated")


def test_moe_refuses_min_types_and_checks_the_gate_column(qm, dev):
    import torch
    NE, E, Fd, T, NU = 8, 256, 256, 2, 2
    s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=1)
    for tk in (F.Q4_K, F.Q2_K, F.IQ1_S):  # (per-block mins, IQ1: no expert types, as the reference's)
        Wk = F.synth_weight(tk, NE * Fd, E, seed=2)
        wk = qm.QWeight(tk, to_dev(Wk, dev), NE * Fd, E)
        with pytest.raises(qm.QMatmulError) as ei:
            qm.moe_grouped(wk, s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"])
        assert ei.value.status == 3  # QM_ERR_TYPE
        if tk == F.Q4_K:
            wk.release()
    sh = torch.zeros((T, E), device=dev)
    with pytest.raises(qm.QMatmulError) as ei:  # (logits have exactly NE columns: no gate logit)
        qm.moe_grouped(s["g"], s["u"], s["d"], NE, s["lgt"], NU, s["aq"], s["asc"], s["out"], s["ws"], sh=sh)
    assert ei.value.status == 2  # QM_ERR_SHAPE
    wk.release()


def test_moe_route_fully_masked_row(qm, dev):
    """A row whose logits are all -inf: the selection is the lowest experts (a stable order) at weight 0, so the
    token receives no expert output -- on the route launch and on the decode kernel's own routing."""
    import torch
    NE, E, Fd, NU = 16, 256, 256, 4
    for T in (2, 6):
        s = _moe_setup(qm, dev, NE, E, Fd, T, NU, F.IQ4_XS, seed=T)
        lg = s["lg"].copy()
        lg[1, :] = -np.inf
        lgt = to_dev(lg, dev)
        ids, wts, _ = qm.moe_route(lgt, NU)
        torch.cuda.synchronize()
        assert list(ids.cpu().numpy()[1]) == [0, 1, 2, 3] and np.all(wts.cpu().numpy()[1] == 0.0)
        qm.moe_grouped(s["g"], s["u"], s["d"], NE, lgt, NU, s["aq"], s["asc"], s["out"], s["ws"])
        torch.cuda.synchronize()
        got = s["out"].cpu().numpy()
        assert np.all(got[1] == 0.0) and np.all(np.isfinite(got))
        s["lg"] = lg
        moe_check(qm, s, (F.IQ4_XS,) * 3, NE, E, Fd, T, NU)
