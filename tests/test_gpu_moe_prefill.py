"""GPU parity of the routed-MoE prefill path: prefill router, device
grouping, grouped gate/up/down on the matrix cores and the token-major
combine, against the CPU oracle (tests mirror
T/Kernels/Prefill/PrefillRouterTests.swift, PrefillMoEGroupingTests.swift,
PrefillGroupedRoutedMoETests+Execution.swift and PrefillMoETests.swift).
Routing indices and the grouping are bit-exact; floating-point outputs are
held to max relative error <= 1e-3 (RelError.compute)."""
import numpy as np
import pytest

import oracle
from edgeexpert_amd import ops, synth
from edgeexpert_amd.runtime import DeviceBuffer
from helpers import bf16_to_f16_exact, from_f16_bits

pytestmark = pytest.mark.gpu
TOL = oracle.Tolerance.north_star


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _oracle_pool(pool_bytes, offs, stride):
    """(pool, stride, offsets) in the argument order of oracle.grouped_route_partials."""
    return pool_bytes, stride, oracle.ExpertOffsets(*[int(offs[k]) for k in synth.OFFSET_ORDER])


# ------------------------------------------------------------- router ----

@pytest.mark.parametrize("T,E,D,k", [(7, 16, 128, 8), (512, 128, 2816, 8), (33, 256, 512, 64)])
def test_prefill_router_matches_per_token_reference(ctx, stream, T, E, D, k):
    # PrefillRouterTests.swift:33-101: block router == per-row router
    W, S, B = synth.int8_matrix(2, f"pr/{E}x{D}", E, D)
    stride = D + 64
    H = np.zeros((T, stride), np.uint16)
    H[:, :D] = synth.f16_vector(2, f"pr/h{T}", T * D).reshape(T, D)
    eff = synth.f16_bits(np.abs(synth.normal(synth.seed_key(2, "pr/eff"), D)) + 0.5)
    gain = synth.f16_bits(synth.uniform24(synth.seed_key(2, "pr/gain"), E, 0.6, 1.4))
    router = ops.Router(_dev(W), _dev(S), _dev(B), E, _dev(eff), _dev(gain))
    idx, w16 = _dev(np.zeros(T * k, np.uint32)), _dev(np.zeros(T * k, np.uint16))
    wf, logits = _dev(np.zeros(T * k, np.float32)), _dev(np.zeros(T * E, np.float32))
    ops.PrefillRouter(ctx).encode_gemma4_block(stream, router, _dev(H), stride, T, D, k, idx, w16, logits,
                                               out_weights_f32=wf)
    stream.sync()
    got_idx = idx.download(np.uint32).reshape(T, k)
    got_w = wf.download(np.float32).reshape(T, k)
    ref_idx, ref_w = oracle.prefill_router(W, S, B, from_f16_bits(H[:, :D]), k, eff=from_f16_bits(eff),
                                           expert_scale=from_f16_bits(gain))
    assert np.array_equal(got_idx, ref_idx)
    # softmax weights move by ~|Δlogit| (fp32 summation-order differences, ~1e-6 of |logit|)
    assert oracle.rel_error(got_w, ref_w) < 1e-4
    lg = logits.download(np.float32).reshape(T, E)
    for t in (0, T - 1):
        ref_l = oracle.router_logits(W, S, B, from_f16_bits(H[t, :D]), from_f16_bits(eff))
        assert oracle.rel_error(lg[t], ref_l) < 1e-5


# ----------------------------------------------------------- grouping ----

def _device_group(ctx, stream, idx, w16, T, k, E):
    n = T * k
    mt = ops.max_tiles(T, k, E)
    bufs = dict(sorted=_dev(np.zeros(n, ops.PAIR_DTYPE)), offsets=_dev(np.zeros(E, np.uint32)),
                counts=_dev(np.zeros(E, np.uint32)), tiles=_dev(np.zeros(mt, ops.TILE_DTYPE)),
                n_tiles=_dev(np.full(ops.GROUP_STATE_BYTES // 4, 77, np.uint32)),
                status=_dev(np.full(1, 77, np.uint32)))
    ops.PrefillMoEGrouping(ctx).encode(stream, _dev(idx), _dev(w16), T, k, E, bufs["sorted"],
                                       bufs["offsets"], bufs["counts"], bufs["tiles"],
                                       bufs["n_tiles"], bufs["status"])
    stream.sync()
    out = {"sorted": bufs["sorted"].download(np.uint8, n * 16).view(ops.PAIR_DTYPE),
           "offsets": bufs["offsets"].download(np.uint32, E), "counts": bufs["counts"].download(np.uint32, E),
           "n_tiles": int(bufs["n_tiles"].download(np.uint32, 1)[0]),
           "state": bufs["n_tiles"].download(np.uint32, ops.GROUP_STATE_BYTES // 4),
           "status": int(bufs["status"].download(np.uint32, 1)[0])}
    out["tiles"] = bufs["tiles"].download(np.uint8, mt * 16).view(ops.TILE_DTYPE)[:out["n_tiles"]]
    return out, bufs


@pytest.mark.parametrize("T,k,E,label", [(512, 8, 128, "zipf"), (32, 8, 128, "t32"), (1, 8, 16, "one"),
                                         (1024, 8, 256, "big"), (4, 3, 6, "kat")])
def test_device_grouping_bit_exact(ctx, stream, T, k, E, label):
    if label == "t32":
        # PrefillMoEGroupingTests.swift:175-203 pressure pattern
        idx = np.array([[(t + r * 7) % 74 for r in range(8)] for t in range(32)], np.uint32)
        w16 = np.arange(T * k, dtype=np.uint16).reshape(T, k)
    elif label == "kat":
        # PrefillMoEGroupingTests.swift:5-53, token-major input
        idx = np.array([[3, 1, 4], [1, 3, 2], [4, 3, 1], [5, 1, 4]], np.uint32)
        w16 = np.arange(10, 22, dtype=np.uint16).reshape(4, 3)
    else:
        idx, w16 = synth.zipf_routing(4, f"dg/{label}", T, E, k)
    got, _ = _device_group(ctx, stream, idx, w16, T, k, E)
    pairs = ops.PrefillRouter.make_token_expert_pairs(idx, w16, T, k)
    ref = oracle.group_pairs(pairs.astype(oracle.PAIR_DTYPE), T, k, E, 16)
    assert got["status"] == 0
    assert got["sorted"].tobytes() == ref["sorted"].tobytes()
    assert np.array_equal(got["offsets"], ref["offsets"])
    assert np.array_equal(got["counts"], ref["counts"])
    # tiles: every expert's run cut into <=128-row tiles, in expert order
    exp_tiles = []
    for e in range(E):
        c = int(ref["counts"][e])
        for s0 in range(0, c, 128):
            exp_tiles.append((e, int(ref["offsets"][e]) + s0, min(128, c - s0), 0))
    assert [tuple(int(v) for v in t) for t in got["tiles"]] == exp_tiles
    if label == "kat":
        assert list(got["sorted"]["expert"]) == [1, 1, 1, 1, 2, 3, 3, 3, 4, 4, 4, 5]
        assert list(got["offsets"]) == [0xFFFFFFFF, 0, 4, 5, 8, 11]


def test_device_grouping_rejects_out_of_range_expert(ctx, stream):
    idx = np.array([[0, 1], [2, 9]], np.uint32)
    got, _ = _device_group(ctx, stream, idx, np.zeros((2, 2), np.uint16), 2, 2, 4)
    assert got["status"] == 8 and got["n_tiles"] == 0          # expertOutOfRange
    assert list(got["counts"]) == [0, 0, 0, 0]


# ----------------------------------------------------- grouped experts ----

def _synthetic_rows(rows, cols, expert, role):
    # PrefillGroupedRoutedMoETests.syntheticRows (PrefillGroupedRoutedMoETests.swift:207-216)
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    return (np.float32(expert + 1) * np.float32(0.001) + np.float32(role + 1) * np.float32(0.003)
            + ((r % 7) - 3).astype(np.float32) * np.float32(0.0004)
            + ((c % 11) - 5).astype(np.float32) * np.float32(0.0002)).astype(np.float32)


def _synthetic_pool(num_experts, d, f):
    # makeSyntheticExpertPool (PrefillGroupedRoutedMoETests.swift:113-175), fp16 scale words
    offsets, stride = synth.expert_layout(d, f, align=256)
    pool = np.zeros(num_experts * stride, np.uint8)
    for e in range(num_experts):
        for role, (proj, rows, cols) in enumerate((("gate", f, d), ("up", f, d), ("down", d, f))):
            W, S, B = oracle.quantize_int4_matrix(_synthetic_rows(rows, cols, e, role))
            for part, arr in (("w", W), ("s", bf16_to_f16_exact(S)), ("b", bf16_to_f16_exact(B))):
                raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
                o = e * stride + offsets[f"{proj}_{part}"]
                pool[o:o + raw.size] = raw
    return pool, offsets, stride


# Fill of output rows no pair writes: a NaN bit pattern no kernel stores (the
# fp16 conversions produce the canonical NaN 0x7E00 at most).
UNWRITTEN = np.uint16(0x7FFF)


def _run_grouped(ctx, stream, pool_bytes, offs, stride, E, idx, w16, hidden16, stride_h, T, k, d, f):
    got, bufs = _device_group(ctx, stream, idx, w16, T, k, E)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    act = _dev(np.full(T * k * f, UNWRITTEN, np.uint16))
    partials = _dev(np.full(T * k * d, UNWRITTEN, np.uint16))
    h2 = _dev(np.zeros(T * d, np.uint16))
    g = ops.PrefillGroupedRoutedMoE(ctx)
    g.encode(stream, pool, bufs["sorted"], bufs["tiles"], bufs["n_tiles"], ops.max_tiles(T, k, E),
             _dev(hidden16), stride_h, d, f, k, act, partials)
    g.encode_reduce_token_major(stream, partials, _dev(w16), h2, T, k, d)
    stream.sync()
    # every pair's act row (sorted position) is written by gate/up
    n = len(got["sorted"])
    left = np.argwhere(act.download(np.uint16).reshape(T * k, f)[:n] == UNWRITTEN)
    assert left.shape[0] == 0, f"{left.shape[0]} act entries unwritten, e.g. (row, feature) {left[:8].tolist()}"
    return got, partials.download(np.uint16), h2.download(np.uint16)


def test_grouped_partials_match_reference_small(ctx, stream):
    # PrefillGroupedRoutedMoETests+Execution.swift:8-103 (d=64, f=64, 3 tokens, top-2, 16 experts)
    d, f, T, k, E = 64, 64, 3, 2, 16
    pool_bytes, offs, stride = _synthetic_pool(E, d, f)
    idx = np.array([[2, 0], [1, 2], [0, 1]], np.uint32)
    w16 = synth.f16_bits(np.array([[0.125, 0.1875]] * 3, np.float32))
    hidden = (((np.arange(T * d) % 17) - 8) * 0.01).astype(np.float16).view(np.uint16)
    got, parts, h2 = _run_grouped(ctx, stream, pool_bytes, offs, stride, E, idx, w16, hidden, d, T, k, d, f)
    ref = oracle.grouped_route_partials(got["sorted"].astype(oracle.PAIR_DTYPE), hidden, d,
                                        *_oracle_pool(pool_bytes, offs, stride), k, d, f, T)
    gp, rp = from_f16_bits(parts), from_f16_bits(ref)
    # The reference's bound (absolute 1.5e-3). These synthetic experts give
    # partials of ~1e-6, inside fp16's subnormal range, so a relative bound is
    # not meaningful here; the config-3 test below holds the 1e-3 relative bar.
    assert np.max(np.abs(gp - rp)) <= 0.0015
    assert np.array_equal(parts == UNWRITTEN, ref == np.float16(-99).view(np.uint16))
    ref_h2 = from_f16_bits(oracle.reduce_token_major(ref, w16.ravel(), T, k, d))
    assert np.max(np.abs(from_f16_bits(h2) - ref_h2)) <= 0.0015


def test_combine_matches_reference(ctx, stream):
    # PrefillMoETests.swift:8-44 (SplitMix64 seed 0x4D0E2026, 3 tokens x top-8 x 64)
    rows, k, d = 3, 8, 64
    r = oracle.SplitMix64(0x4D0E2026)
    partials = r.uniforms(rows * k * d, -2.0, 2.0).astype(np.float16).view(np.uint16)
    weights = r.uniforms(rows * k, -1.0, 1.0).astype(np.float16).view(np.uint16)
    h2 = _dev(np.full(rows * d, np.float16(-19.0).view(np.uint16), np.uint16))
    ops.PrefillGroupedRoutedMoE(ctx).encode_reduce_token_major(stream, _dev(partials), _dev(weights), h2,
                                                               rows, k, d)
    stream.sync()
    got = from_f16_bits(h2.download(np.uint16))
    ref = from_f16_bits(oracle.reduce_token_major(partials, weights, rows, k, d))
    assert np.max(np.abs(got - ref)) <= 2e-3                        # the reference's bound
    assert oracle.rel_error(got, ref) < TOL


def test_grouped_moe_baseline_config3_sampled(ctx, stream):
    # 512 tokens x top-8 over 128 experts (D=2816, F=704),
    # Zipf(1.1) popularity; oracle on the pairs of 12 sampled tokens.
    T, k, E, d, f = 512, 8, 128, 2816, 704
    pool_bytes, offs, stride = synth.expert_pool(0, "c3/experts", E, d, f)
    idx, w16 = synth.zipf_routing(0, "c3/route", T, E, k)
    hidden = synth.f16_vector(0, "c3/x", T * d)
    got, parts, h2 = _run_grouped(ctx, stream, pool_bytes, offs, stride, E, idx, w16, hidden, d, T, k, d, f)
    assert got["status"] == 0
    toks = np.array([0, 1, 77, 128, 255, 256, 300, 383, 400, 450, 510, 511])
    sel = got["sorted"][np.isin(got["sorted"]["token"], toks)]
    ref = oracle.grouped_route_partials(sel.astype(oracle.PAIR_DTYPE), hidden, d,
                                        *_oracle_pool(pool_bytes, offs, stride), k, d, f, T)
    # every (token, rank) slot has a pair here: no unit of the down launch was skipped
    assert not np.any(parts == UNWRITTEN)
    gp, rp = from_f16_bits(parts).reshape(T, k, d), from_f16_bits(ref).reshape(T, k, d)
    rel = oracle.rel_error(gp[toks], rp[toks])
    assert rel < TOL, f"partials rel={rel}"
    ref_h2 = from_f16_bits(oracle.reduce_token_major(ref, w16.ravel(), T, k, d)).reshape(T, d)
    rel = oracle.rel_error(from_f16_bits(h2).reshape(T, d)[toks], ref_h2[toks])
    assert rel < TOL, f"h2 rel={rel}"
    # and the first and last pair of every active expert: every grouping tile,
    # both halves of the wide ones and every unit class is checked
    srt = got["sorted"]
    ends = sorted({i for e in np.unique(srt["expert"])
                   for i in (int(np.flatnonzero(srt["expert"] == e)[0]), int(np.flatnonzero(srt["expert"] == e)[-1]))})
    sel = srt[ends]
    ref2 = oracle.grouped_route_partials(sel.astype(oracle.PAIR_DTYPE), hidden, d,
                                         *_oracle_pool(pool_bytes, offs, stride), k, d, f, T)
    slots = sel["token"].astype(np.int64) * k + sel["rank"].astype(np.int64)
    rel = oracle.rel_error(gp.reshape(T * k, d)[slots], from_f16_bits(ref2).reshape(T * k, d)[slots])
    assert rel < TOL, f"per-expert partials rel={rel}"


@pytest.mark.parametrize("bits", [4, 3])
def test_grouped_tile_and_stream_split(ctx, stream, bits):
    # experts whose grouping tiles fall on both sides of the stream cut (32
    # pairs): 1, 16, 17, 32 pairs (the weight stream, one and two 16-pair
    # sub-tiles), 33, 72, 100 (the MFMA tile), 129 (a full tile plus a
    # one-pair tile on the stream). f = 192 leaves a partial block of
    # features (gate/up) and a half-filled last 128-code k-tile (down); every
    # pair is checked against the oracle.
    d, f, k, E = 256, 192, 2, 8
    counts = [129, 33, 32, 17, 16, 1, 72, 100]
    T = sum(counts) // k
    order = np.repeat(np.arange(E, dtype=np.uint32), counts)
    idx = np.stack([order[:T], order[T:]], axis=1)
    assert np.all(idx[:, 0] != idx[:, 1])
    w16 = synth.f16_bits(synth.uniform24(synth.seed_key(9, "split/w"), T * k, 0.1, 0.9)).reshape(T, k)
    pool_bytes, offs, stride = synth.expert_pool(9, f"split/b{bits}", E, d, f, bits=bits)
    hidden = synth.f16_vector(9, "split/x", T * d)
    got, bufs = _device_group(ctx, stream, idx, w16, T, k, E)
    assert got["status"] == 0
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs, weight_bits=bits)
    act = _dev(np.zeros(T * k * f, np.uint16))
    partials = _dev(np.full(T * k * d, np.float16(-77).view(np.uint16), np.uint16))
    ops.PrefillGroupedRoutedMoE(ctx).encode(stream, pool, bufs["sorted"], bufs["tiles"], bufs["n_tiles"],
                                            ops.max_tiles(T, k, E), _dev(hidden), d, d, f, k, act, partials)
    stream.sync()
    ref = oracle.grouped_route_partials(got["sorted"].astype(oracle.PAIR_DTYPE), hidden, d,
                                        *_oracle_pool(pool_bytes, offs, stride), k, d, f, T, bits=bits)
    gp, rp = from_f16_bits(partials.download(np.uint16)).reshape(T * k, d), from_f16_bits(ref).reshape(T * k, d)
    for e, c in enumerate(counts):
        rows = [int(p["token"]) * k + int(p["rank"]) for p in got["sorted"] if p["expert"] == e]
        assert len(rows) == c
        rel = oracle.rel_error(gp[rows], rp[rows])
        assert rel < TOL, f"expert {e} ({c} pairs): rel={rel}"


def _repack_misaligned(pool_bytes, offs, stride, E, d, f):
    # the same experts with every scale and bias array at a 2-byte (not
    # 16-byte) aligned offset, weight arrays still 16-byte aligned
    sizes = {"gate_w": f * d // 2, "gate_s": f * (d // 64) * 2, "gate_b": f * (d // 64) * 2,
             "up_w": f * d // 2, "up_s": f * (d // 64) * 2, "up_b": f * (d // 64) * 2,
             "down_w": d * f // 2, "down_s": d * (f // 64) * 2, "down_b": d * (f // 64) * 2}
    new, cur = {}, 0
    for name in synth.OFFSET_ORDER:
        cur = (cur + 15) // 16 * 16 + (2 if name.endswith(("_s", "_b")) else 0)
        new[name] = cur
        cur += sizes[name]
    new_stride = (cur + 255) // 256 * 256
    out = np.zeros(E * new_stride, np.uint8)
    for e in range(E):
        for name in synth.OFFSET_ORDER:
            src = e * stride + offs[name]
            out[e * new_stride + new[name]:e * new_stride + new[name] + sizes[name]] = pool_bytes[src:src + sizes[name]]
    return out, new, new_stride


def test_grouped_table_forms_agree(ctx, stream):
    # 16-byte aligned scale/bias arrays take the launches that stage each
    # unit's scale/bias table through registers, 2-byte aligned ones the
    # launches that copy it through a loop: the same table, so the same bits
    T, k, E, d, f = 128, 8, 32, 512, 256
    pool_bytes, offs, stride = synth.expert_pool(11, "tables/experts", E, d, f)
    idx, w16 = synth.zipf_routing(11, "tables/route", T, E, k)
    hidden = synth.f16_vector(11, "tables/x", T * d)
    mis_bytes, mis_offs, mis_stride = _repack_misaligned(pool_bytes, offs, stride, E, d, f)
    assert all(mis_offs[n] % 16 == 2 for n in synth.OFFSET_ORDER if n.endswith(("_s", "_b")))
    got, parts, h2 = _run_grouped(ctx, stream, pool_bytes, offs, stride, E, idx, w16, hidden, d, T, k, d, f)
    _, parts_m, h2_m = _run_grouped(ctx, stream, mis_bytes, mis_offs, mis_stride, E, idx, w16, hidden, d, T, k, d, f)
    assert got["status"] == 0 and not np.any(parts == UNWRITTEN)
    assert np.array_equal(parts, parts_m) and np.array_equal(h2, h2_m)
    ref = oracle.grouped_route_partials(got["sorted"].astype(oracle.PAIR_DTYPE), hidden, d,
                                        *_oracle_pool(pool_bytes, offs, stride), k, d, f, T)
    rel = oracle.rel_error(from_f16_bits(parts), from_f16_bits(ref))
    assert rel < TOL, f"partials rel={rel}"


def test_grouped_schedule_at_tile_bound(ctx, stream):
    # 8192 pairs over 256 experts: the tile bound (TFQ_MOE_MAX_TILES = 320)
    # and a work list of several units per resident block in both launches;
    # every pair against the oracle and no output row left unwritten.
    T, k, E, d, f = 1024, 8, 256, 128, 128
    assert ops.max_tiles(T, k, E) == 320
    pool_bytes, offs, stride = synth.expert_pool(5, "bound/experts", E, d, f)
    idx, w16 = synth.zipf_routing(5, "bound/route", T, E, k)
    hidden = synth.f16_vector(5, "bound/x", T * d)
    got, parts, _ = _run_grouped(ctx, stream, pool_bytes, offs, stride, E, idx, w16, hidden, d, T, k, d, f)
    assert got["status"] == 0
    assert not np.any(parts == UNWRITTEN)
    ref = oracle.grouped_route_partials(got["sorted"].astype(oracle.PAIR_DTYPE), hidden, d,
                                        *_oracle_pool(pool_bytes, offs, stride), k, d, f, T)
    rel = oracle.rel_error(from_f16_bits(parts), from_f16_bits(ref))
    assert rel < TOL, f"partials rel={rel}"


def test_grouped_repeat_on_one_grouping(ctx, stream):
    # the grouped launches take their units from counters in the grouping
    # state and leave them zero: two calls on one grouping give the same
    # bits, every row written both times
    T, k, E, d, f = 256, 8, 64, 256, 128
    pool_bytes, offs, stride = synth.expert_pool(6, "repeat/experts", E, d, f)
    idx, w16 = synth.zipf_routing(6, "repeat/route", T, E, k)
    hidden = _dev(synth.f16_vector(6, "repeat/x", T * d))
    got, bufs = _device_group(ctx, stream, idx, w16, T, k, E)
    assert got["status"] == 0 and np.all(got["state"][1:] == 0)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    outs = []
    for _ in range(2):
        act = _dev(np.full(T * k * f, UNWRITTEN, np.uint16))
        partials = _dev(np.full(T * k * d, UNWRITTEN, np.uint16))
        ops.PrefillGroupedRoutedMoE(ctx).encode(stream, pool, bufs["sorted"], bufs["tiles"], bufs["n_tiles"],
                                                ops.max_tiles(T, k, E), hidden, d, d, f, k, act, partials)
        stream.sync()
        state = bufs["n_tiles"].download(np.uint32, ops.GROUP_STATE_BYTES // 4)
        assert state[0] == got["n_tiles"] and np.all(state[1:] == 0), state
        outs.append((act.download(np.uint16), partials.download(np.uint16)))
    for a, p in outs:
        assert not np.any(a == UNWRITTEN) and not np.any(p == UNWRITTEN)
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_moe_prefill_end_to_end(ctx, stream):
    # router -> grouping -> grouped experts -> combine through one call
    T, k, E, d, f = 64, 8, 32, 512, 256
    pool_bytes, offs, stride = synth.expert_pool(1, "pf/experts", E, d, f)
    Wr, Sr, Br = synth.int8_matrix(1, "pf/router", E, d)
    hidden = synth.f16_vector(1, "pf/x", T * d)
    router = ops.Router(_dev(Wr), _dev(Sr), _dev(Br), E)
    pool = ops.ExpertPool(_dev(pool_bytes), stride, E, offs)
    wsb = ops.moe_prefill_workspace_bytes(T, k, E, d, f)
    ws = DeviceBuffer(wsb)
    idx, w16, h2 = _dev(np.zeros(T * k, np.uint32)), _dev(np.zeros(T * k, np.uint16)), _dev(np.zeros(T * d, np.uint16))
    ops.moe_prefill(ctx, stream, router, pool, _dev(hidden), d, T, d, f, k, h2, idx, w16, ws, wsb)
    stream.sync()
    ref_idx, ref_w = oracle.prefill_router(Wr, Sr, Br, from_f16_bits(hidden).reshape(T, d), k)
    got_idx = idx.download(np.uint32).reshape(T, k)
    assert np.array_equal(got_idx, ref_idx)
    w_dev = w16.download(np.uint16)
    pairs = ops.PrefillRouter.make_token_expert_pairs(got_idx, w_dev, T, k)
    grp = oracle.group_pairs(pairs.astype(oracle.PAIR_DTYPE), T, k, E, 16)
    ref = oracle.grouped_route_partials(grp["sorted"], hidden, d, *_oracle_pool(pool_bytes, offs, stride),
                                        k, d, f, T)
    ref_h2 = from_f16_bits(oracle.reduce_token_major(ref, w_dev, T, k, d))
    rel = oracle.rel_error(from_f16_bits(h2.download(np.uint16)), ref_h2)
    assert rel < TOL, f"rel={rel}"
