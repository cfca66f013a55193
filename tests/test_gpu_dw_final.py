"""The weight-gradient group that assembles its own gradients
(ppo_gemm_f32_dw_group_final) against the grouped launch followed by the
gradient-assembly launch (ppo_gemm_f32_dw_group + ppo_grad_reduce) on the same
inputs: the same gradient bits, the same total squared norm, the other
segments reduced in the same launch, the arrival counters left at zero."""
import ctypes
import struct

import numpy as np
import pytest
import torch

from boonta_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def st():
    return torch.cuda.current_stream().cuda_stream


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def tables(segs, slot0, flags=0):
    """Device segment / chunk tables in the reduce's layout (the learner's
    packing): (SEGS, CHUNKS, nchunks, nfew, nwide); flags 1 rounds the sums
    to bf16."""
    lib = _lib.load()
    chunk, wide_chunk = lib.ppo_grad_reduce_chunk_elems(), lib.ppo_grad_reduce_wide_chunk_elems()
    few_parts, wide_parts = lib.ppo_grad_reduce_few_parts(), lib.ppo_grad_reduce_wide_parts()
    few, many, wide = [], [], []
    for i, (_, _, c, _, n) in enumerate(segs):
        dst = few if n <= few_parts else wide if n > wide_parts else many
        for start in range(0, c, wide_chunk if dst is wide else chunk):
            dst.append(struct.pack("<iiq", i, slot0 + len(few) + len(many) + len(wide), start))
    seg_bytes = b"".join(struct.pack("<QQqqii", d, s, c, ps, n, flags) for d, s, c, ps, n in segs)
    chunks = few + many + wide
    t = lambda b: torch.tensor(list(b) or [0], dtype=torch.uint8, device=DEV)
    return t(seg_bytes), t(b"".join(chunks)), len(chunks), len(few), len(wide)


# (rows of A, M, N, K, splits, gathered, gradient rows, with bias): the paired
# towers' first layers over a zero-padded 88-column input (87 gradient rows),
# their 256-wide later layers, and ragged problems (K off the stage depth, M
# and N off the tile) with the other supported split counts
SHAPES = [(4096, 88, 256, 2048, 16, True, 87, True), (4096, 88, 256, 2048, 16, True, 87, True),
          (2048, 256, 256, 2048, 8, False, 256, True), (2048, 256, 256, 2048, 8, False, 256, True),
          (1000, 68, 132, 1000, 3, False, 66, True), (700, 36, 200, 700, 12, True, 36, False),
          (300, 64, 64, 300, 1, False, 64, True), (900, 128, 72, 900, 6, False, 125, True)]
# other segments (elements, partials): wide, few and many partials
OTHER = [(512, 128), (256, 3), (1000, 20), (4, 200)]


def make_case(rng, shapes=SHAPES):
    probs = []
    for R, M, N, K, sp, gathered, grows, bias in shapes:
        A = dev(rng.normal(size=(R, M)).astype(np.float32))
        idx = dev(rng.permutation(R)[:K].astype(np.int32)) if gathered else None
        B = dev(rng.normal(size=(K, N)).astype(np.float32))
        probs.append((A, idx, B, M, N, K, sp, grows, bias))
    other = [dev(rng.normal(size=(n, c)).astype(np.float32)) for c, n in OTHER]
    return probs, other


def group_args(probs, C, bg):
    L = len(probs)
    vp = lambda xs: (ctypes.c_void_p * L)(*xs)
    i64 = lambda xs: (ctypes.c_int64 * L)(*xs)
    i32 = lambda xs: (ctypes.c_int * L)(*xs)
    return [vp([p[0].data_ptr() for p in probs]), i64([p[3] for p in probs]),
            vp([None if p[1] is None else p[1].data_ptr() for p in probs]), vp([p[2].data_ptr() for p in probs]),
            i64([p[4] for p in probs]), vp([c.data_ptr() for c in C]), i64([p[4] for p in probs]),
            i32([p[3] for p in probs]), i32([p[4] for p in probs]), i32([p[5] for p in probs]),
            i32([p[6] for p in probs]), i64([p[3] * p[4] for p in probs]), vp([b.data_ptr() for b in bg])]


def reference(probs, other):
    """Grouped partials, then the reduce over every segment (slots 0..)."""
    C = [torch.full((p[6], p[3], p[4]), float("nan"), device=DEV) for p in probs]
    bg = [torch.full((p[6], p[4]), float("nan"), device=DEV) for p in probs]
    args = group_args(probs, C, bg)
    _lib.call("ppo_gemm_f32_dw_group", st(), len(probs), *[ctypes.addressof(a) for a in args])
    G = [torch.full((p[7], p[4]), float("nan"), device=DEV) for p in probs]
    Gb = [torch.full((p[4],), float("nan"), device=DEV) for p in probs]
    O = [torch.full((c,), float("nan"), device=DEV) for c, _ in OTHER]
    segs = []
    for p, c, b, g, gb in zip(probs, C, bg, G, Gb):
        segs.append((g.data_ptr(), c.data_ptr(), p[7] * p[4], p[3] * p[4], p[6]))
        if p[8]:
            segs.append((gb.data_ptr(), b.data_ptr(), p[4], p[4], p[6]))
    for o, src, (c, n) in zip(O, other, OTHER):
        segs.append((o.data_ptr(), src.data_ptr(), c, c, n))
    SEGS, CH, nch, nfew, nwide = tables(segs, 0)
    SQ = torch.zeros(nch, dtype=torch.float64, device=DEV)
    _lib.call("ppo_grad_reduce", st(), SEGS.data_ptr(), CH.data_ptr(), nch, nfew, nwide, SQ.data_ptr())
    return [host(g) for g in G], [host(b) for b in Gb], [host(o) for o in O], float(host(SQ).sum())


def finished(probs, other, counters=None):
    """The finishing launch over the same problems and other segments."""
    L = len(probs)
    lib = _lib.load()
    T = lib.ppo_gemm_f32_dw_final_slots(L, (ctypes.c_int * L)(*[p[3] for p in probs]),
                                        (ctypes.c_int * L)(*[p[4] for p in probs]))
    assert T == sum(-(-p[3] // 64) * -(-p[4] // 64) for p in probs)
    # one counter per tile, then eight per tile for the two-level sums
    C = [torch.full((p[6], p[3], p[4]), float("nan"), device=DEV) for p in probs]
    bg = [torch.full((p[6], p[4]), float("nan"), device=DEV) for p in probs]
    # one guard row after each gradient: the rows past g_rows stay untouched
    G = [torch.full((p[7] + 1, p[4]), float("nan"), device=DEV) for p in probs]
    Gb = [torch.full((p[4],), float("nan"), device=DEV) for p in probs]
    O = [torch.full((c,), float("nan"), device=DEV) for c, _ in OTHER]
    segs = [(o.data_ptr(), src.data_ptr(), c, c, n) for o, src, (c, n) in zip(O, other, OTHER)]
    SEGS, CH, nch, nfew, nwide = tables(segs, T)
    SQ = torch.full((T + nch,), float("nan"), dtype=torch.float64, device=DEV)
    if counters is None:
        counters = torch.zeros(9 * T, dtype=torch.int32, device=DEV)
    args = group_args(probs, C, bg)
    vp = lambda xs: (ctypes.c_void_p * L)(*xs)
    fin = [vp([g.data_ptr() for g in G]), (ctypes.c_int64 * L)(*[p[4] for p in probs]),
           (ctypes.c_int * L)(*[p[7] for p in probs]),
           vp([b.data_ptr() if p[8] else None for b, p in zip(Gb, probs)])]
    rc = _lib.call("ppo_gemm_f32_dw_group_final", st(), L, *[ctypes.addressof(a) for a in args + fin],
                   counters.data_ptr(), SQ.data_ptr(), SEGS.data_ptr(), CH.data_ptr(), nch, nfew, nwide)
    assert rc == 0
    return [host(g) for g in G], [host(b) for b in Gb], [host(o) for o in O], host(SQ), counters


def same_bits(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def check(probs, other, counters=None):
    G1, B1, O1, sq1 = reference(probs, other)
    G2, B2, O2, SQ2, counters = finished(probs, other, counters)
    for k, p in enumerate(probs):
        assert same_bits(G1[k], G2[k][:p[7]]), f"problem {k}: gradient differs"
        assert np.isnan(G2[k][p[7]]).all(), f"problem {k}: a row past the gradient was written"
        if p[8]:
            assert same_bits(B1[k], B2[k]), f"problem {k}: bias gradient differs"
        else:
            assert np.isnan(B2[k]).all()
    for k in range(len(OTHER)):
        assert same_bits(O1[k], O2[k]), f"other segment {k} differs"
    assert not np.isnan(SQ2).any(), "a norm slot was not written"
    np.testing.assert_allclose(SQ2.sum(), sq1, rtol=1e-12)
    assert not host(counters).any(), "arrival counters not left at zero"
    return counters


def test_final_group_matches_the_group_and_reduce_launches():
    rng = np.random.default_rng(3)
    probs, other = make_case(rng)
    counters = check(probs, other)
    # a second call with new values through the same counters
    probs2, other2 = make_case(rng)
    check(probs2, other2, counters)
    # a float64 check of the gathered first problem
    A, idx, B, M, N, K, sp, grows, _ = probs[0]
    G, _, _, _, _ = finished(probs, other)
    want = (host(A).astype(np.float64)[host(idx)].T @ host(B).astype(np.float64))[:grows]
    np.testing.assert_allclose(G[0][:grows], want, rtol=2e-5, atol=2e-4)


# two-level sums: 64 splits (the discrete Anakin workload's first layer: 400 x 256 over gathered rows)
# and 32 splits (a ragged problem)
SHAPES2 = [(8192, 400, 256, 4096, 64, True, 400, True), (3000, 128, 136, 2048, 32, False, 120, True),
           (2048, 256, 256, 2048, 8, False, 256, True)]


def test_final_group_two_level_sums_match_the_group_and_reduce_launches():
    rng = np.random.default_rng(9)
    counters = None
    for _ in range(2):
        probs, other = make_case(rng, SHAPES2)
        counters = check(probs, other, counters)


def test_final_group_rejects_unsupported_shapes():
    rng = np.random.default_rng(4)
    probs, other = make_case(rng)
    L = 1
    p = probs[2]
    C = torch.zeros((p[6], p[3], p[4]), device=DEV)
    bg = torch.zeros((p[6], p[4]), device=DEV)
    G = torch.zeros((p[3], p[4]), device=DEV)
    cnt = torch.zeros(9 * 16, dtype=torch.int32, device=DEV)
    SQ = torch.zeros(16, dtype=torch.float64, device=DEV)

    def call(splits=p[6], grows=p[7], K=p[5], idx=None):
        q = (p[0], idx, p[2], p[3], p[4], K, splits, grows, True)
        args = group_args([q], [C], [bg])
        fin = [(ctypes.c_void_p * L)(G.data_ptr()), (ctypes.c_int64 * L)(p[4]), (ctypes.c_int * L)(grows),
               (ctypes.c_void_p * L)(None)]
        return _lib.load().ppo_gemm_f32_dw_group_final(
            ctypes.c_void_p(st()), L, *[ctypes.addressof(a) for a in args + fin], ctypes.c_void_p(cnt.data_ptr()),
            ctypes.c_void_p(SQ.data_ptr()), None, None, 0, 0, 0)

    assert call(splits=5) != 0          # a split count without a compiled sum
    assert call(grows=p[3] + 1) != 0    # more gradient rows than the problem's
    assert call(grows=0) != 0
    gidx = dev(np.arange(p[5], dtype=np.int32))
    assert call(splits=2, idx=gidx) != 0   # a gathered split of 1024 rows (at most 512)
    torch.cuda.synchronize()

