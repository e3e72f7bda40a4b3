"""CPU emulation of the HIP kernels' tile indexing at the benchmarked layer shapes.

The index arithmetic of the kernels that tile these shapes is restated here in NumPy over every
workgroup and thread, and every address they form is checked against the buffer it addresses:
the XCD-grouped tile order (kanforge_amd/csrc/kf_gemm.h, xcd_tile_grouped) must visit each tile
exactly once, also when the GEMM core's tail split (kf_gemm_nt.hip) runs whole rounds and tail
tiles as two launches; the tail's compact partial tiles and their reduction stay inside the
workspace the planner sizes; the B-spline P epilogue's LDS regions (kf_kernels.h, p8_kernel)
fit its allocation (kf_abi_p.hip, launch_p8) and its reads stay in the sums it wrote; the wide F
route (f_wide_kernel) and the feature pass (phi_block_kernel) stay inside LDS and their arrays.
A restatement checks the arithmetic as written in the sources, the GPU tests check the results.
"""

import numpy as np
import pytest

# shapes: the GEMM core's (M, N, K) of the FFN workloads and the headline (see bench.py)
GEMM_SHAPES = [
    (3072, 768 * 11, 16384), (768, 3072 * 11, 16384),  # B-spline FFN weight gradients (tail split)
    (16384, 3072, 768 * 11), (16384, 768, 3072 * 11),  # B-spline FFN forward
    (16384, 3072, 768), (16384, 768, 3072), (3072, 768, 16384), (768, 3072, 16384),  # GR-KAN
    (3072, 768 * 11, 512), (768, 3072 * 11, 512),  # the 512-token parity tests
    (300, 265 * 11, 1024), (8192, 3072, 768 * 9),
    (8192, 768, 3072), (3072, 768, 8192),  # the fused SiLU base branch's g W and g^T silu(x)
]


def xcd_tile_grouped(g, n_m, n_n, GM=8):
    """kf_gemm.h xcd_tile_grouped, vectorised over workgroup ids g."""
    g = np.asarray(g, dtype=np.int64)
    total = n_m * n_n
    logical = (g % 8) * (total // 8) + g // 8 if total % 8 == 0 else g
    per_group = GM * n_n
    first_m = (logical // per_group) * GM
    gm = np.minimum(n_m - first_m, GM)
    r = logical % per_group
    return first_m + r % gm, r // gm


def pick_gemm(M, N, S):
    """kf_gemm_nt.hip pick_gemm: (tn, nz, tail_nz, full, rem)."""
    best, best_t = (3, 1, 0, 0, 0), 1e300
    for tn in (3, 2, 1):
        tiles = ((M + 255) // 256) * ((N + 128 * tn - 1) // (128 * tn))
        t_stage = 256.0 * 128 * tn * 64 * 2 / (4.0e12 if tn == 1 else 4.7e12)
        for nz in (1, 2, 3, 4, 6, 8, 10, 12, 16, 24, 32):
            if nz > S:
                break
            wg, s_per = tiles * nz, (S + nz - 1) // nz
            t = ((wg + 255) // 256) * s_per * t_stage + (nz * M * N * 8.0 / 5e12 if nz > 1 else 0.0)
            if t < best_t * 0.98:
                best, best_t = (tn, nz, 0, 0, 0), t
        full = tiles // 256 * 256
        rem = tiles - full
        if full == 0 or rem == 0:
            continue
        for tz in (2, 4, 8, 16, 32):
            if tz > S or rem * tz > 256:
                break
            t = (full // 256) * S * t_stage + ((S + tz - 1) // tz) * t_stage + tz * rem * 256 * 128 * tn * 8.0 / 5e12 + 5e-6
            if t < best_t * 0.98:
                best, best_t = (tn, 1, tz, full, rem), t
    return best


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_tiles_each_visited_once_and_partials_in_bounds(M, N, K):
    S = K // 64
    tn, nz, tz, full, rem = pick_gemm(M, N, S)
    BM, BN = 256, 128 * tn
    n_m, n_n = (M + BM - 1) // BM, (N + BN - 1) // BN
    tiles = n_m * n_n
    launches = [(0, tiles)] if not tz else [(0, full), (full, rem)]
    seen = np.zeros((n_m, n_n), dtype=np.int64)
    for tile0, count in launches:
        tm, tnn = xcd_tile_grouped(tile0 + np.arange(count), n_m, n_n)
        assert (tm >= 0).all() and (tm < n_m).all() and (tnn >= 0).all() and (tnn < n_n).all()
        np.add.at(seen, (tm, tnn), 1)
    assert (seen == 1).all(), "a tile is missed or visited twice"
    # copies: rows past M / N repeat the last row, stages run to the end of the reduction
    m0 = np.arange(n_m) * BM
    assert (np.minimum(m0[:, None] + np.arange(BM), M - 1) < M).all()
    splits = tz if tz else nz
    s_per = (S + splits - 1) // splits
    assert (np.minimum(np.arange(splits) * s_per + s_per, S) * 64 <= K).all()
    if tz:
        # compact partials: workgroup (blockIdx.x < rem, z < tz) writes its whole BM x BN tile at
        # (z rem + blockIdx.x) BM BN; the 16-byte chunk (row, ch) of pass ps is at
        # (ps 64 + row) BN + 4 ch; gemm_tail_reduce reads (z rem + t) BM BN + r BN + c, c < BN
        ws_floats = tz * rem * BM * BN
        z, bx = np.meshgrid(np.arange(tz), np.arange(rem), indexing="ij")
        base = (z * rem + bx) * BM * BN
        last_chunk = (3 * 64 + 63) * BN + (BN // 4 - 1) * 4
        assert base.max() + last_chunk + 4 <= ws_floats
        t = np.arange(rem)
        assert ((tz - 1) * rem + t.max()) * BM * BN + (BM - 1) * BN + BN - 4 + 4 <= ws_floats
        # the reduce's tiles are the tail launch's tiles, in the same order
        tm_r, tn_r = xcd_tile_grouped(full + t, n_m, n_n)
        tm_l, tn_l = xcd_tile_grouped(full + np.arange(rem), n_m, n_n)
        assert (tm_r == tm_l).all() and (tn_r == tn_l).all()


@pytest.mark.parametrize("n_in,n_out,grid,k", [(3072, 768, 8, 3), (768, 3072, 8, 3), (265, 300, 8, 3), (64, 64, 5, 3)])
def test_bspline_p_epilogue_lds_regions(n_in, n_out, grid, k):
    """p8_kernel<BSPLINE, NF = 12, TN = 3, RB = 128>: sums red [NF][RPASS][RP], then the knot rows
    kcs [TI][n_knots], kps [TI][n_knots + 2k] and kus [TI][2], all inside launch_p8's LDS."""
    NF, TN, RB = 12, 3, 128
    BM, BN = 256, 128 * TN
    TI, RPASS = BN // NF, 64
    RP, K, nk = TI + 1, grid + k, grid + 2 * k + 1
    lds_ops = 2 * (256 + NF * TI) * RB
    lds_epi = NF * RPASS * RP * 4 + TI * (2 * nk + 2 * k + 2) * 4
    lds = max(lds_ops, lds_epi)
    assert lds <= 160 * 1024
    # the sums: wave (wm, wn), accumulator (a, t, r), lane -> red[(f RPASS + rbase + row) RP + il];
    # in every pass the written slots are exactly the (feature, row, input) slots, each once
    lane = np.arange(64)
    expect = np.sort(((np.arange(NF)[:, None, None] * RPASS + np.arange(RPASS)[None, :, None]) * RP
                      + np.arange(TI)[None, None, :]).ravel())
    for ps in range(BM // RPASS):
        written = []
        for wave in range(8):
            wm, wn = wave & 1, wave >> 1
            for a in range(4):
                if (wm * 128 + a * 32) // RPASS != ps:
                    continue
                rbase = (wm * 128 + a * 32) % RPASS
                for t in range(TN):
                    col = (TN * wn + t) * 32 + (lane & 31)
                    f, il = col // TI, col % TI
                    for r in range(16):
                        row = (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5)
                        written.append((f * RPASS + rbase + row) * RP + il)
        got = np.sort(np.concatenate(written))
        assert got.shape == expect.shape and (got == expect).all(), f"pass {ps}: sums layout is not a bijection"
    # knot rows and spacing after the sums (floats)
    kcs0 = NF * RPASS * RP
    kus_end = kcs0 + TI * nk + TI * (nk + 2 * k) + 2 * TI
    assert kus_end * 4 <= lds
    # the support reads: red[((base + r) RPASS + row) RP + il + u] with 0 <= base + r < K <= NF
    assert K <= NF
    assert ((K - 1) * RPASS + RPASS - 1) * RP + TI - 1 < NF * RPASS * RP
    # each thread's two inputs are fixed over the passes (512 a multiple of TI / 2), and the
    # item rows stay inside a pass
    EPT = RPASS * TI // 2 // 512
    tid = np.arange(512)
    assert 512 % (TI // 2) == 0 and EPT * 512 == RPASS * TI // 2
    rows = (tid[None, :] + 512 * np.arange(EPT)[:, None]) // (TI // 2)
    assert rows.max() < RPASS


@pytest.mark.parametrize("n_in,n_out,KM,K", [(2, 64, 8, 7), (4, 300, 16, 16), (3, 9, 4, 4), (1, 4096, 12, 11)])
def test_f_wide_kernel_indexing(n_in, n_out, KM, K):
    """f_wide_kernel<T, KM, RB = 128>: phs [RB][4 KM] in LDS, lane = output of a 64-output chunk."""
    RB, FR = 128, 4 * KM
    assert n_in <= 4 and K <= KM
    e = np.arange(RB * 4)
    r, i = e // 4, e % 4
    slot = i[:, None] * KM + np.arange(KM)[None, :]
    assert slot.max() < FR and r.max() < RB
    assert RB * FR * 4 <= 64 * 1024
    o = np.arange((n_out + 63) // 64)[:, None] * 64 + np.arange(64)[None, :]
    j = np.arange(FR)
    ok = (o[..., None] < n_out) & ((j // KM) < n_in) & ((j % KM) < K)
    idx = (o[..., None] * n_in + j // KM) * K + j % KM
    assert idx[ok].max() < n_out * n_in * K


@pytest.mark.parametrize("n_in,K", [(768, 11), (3072, 11), (265, 11), (64, 8), (33, 16)])
def test_phi_block_kernel_indexing(n_in, K):
    """phi_block_kernel: 32 inputs x 64 rows per block, row segments of the block's inputs in LDS
    (pitch rpb bytes), knot rows after them; 16-byte row chunks back to phi[b][i K + k]."""
    ROWS, T = 64, 2  # bf16
    rpb = (32 * K * T + 15) // 16 * 16 + 16
    nk, kd = K + 4, 3
    lds = ROWS * rpb + 32 * (2 * nk + 2 * kd) * 4
    assert lds <= 160 * 1024
    # the support writes seg[base + r] with 0 <= base + r < K for lanes il < 32
    il = np.arange(32)
    byte = (il[:, None] * K + np.arange(K)[None, :]) * T
    assert byte.max() + T <= rpb - 16  # inside the row's segment copy
    # stores: chunk q < nv of a row covers elements q VW .. q VW + VW - 1 < n = ni K
    VW = 16 // T
    for i0 in range(0, n_in, 32):
        n = min(n_in - i0, 32) * K
        nv = n // VW
        if nv:
            assert (nv - 1) * VW + VW <= n
            assert (i0 * K + n) <= n_in * K


def f_rega_schedule(NT, n_tp, n_chunks, NBUF=4, base=True):
    """Events of f_rega_kernel (kf_kernels.h) in program order, restated from its loops: the
    chunk copy issues of copy_stage (with the carrier state machine zg_next / zx_next), the seeds
    (SEED2 in a stage's first half, SEEDN in its second), the base-feature reads (BASE2 first
    half, BASEN second half) and the mid-stage barriers. Each event is (stage, half, kind, chunk);
    half 0 runs before the stage's barrier, half 1 after it; the prologue is stage -1 (its copies
    before its barrier, the first seed after). A copy event carries the group g it rides with."""
    ODD = NT % 2 == 1
    P = NT // 2 if NT > 0 and not ODD else n_tp // 2
    S = n_chunks * n_tp // 2
    ev = []
    st = {"zg": P if not ODD else NT // 2, "zx": 1}

    def copy_stage(stage_issued, g):
        if g == st["zg"]:
            if st["zx"] < n_chunks:
                ev.append((stage_issued, 0, "copy", st["zx"], g))
            st["zg"] += P if not ODD else (NT // 2 + 1 if st["zx"] & 1 else NT // 2)
            st["zx"] += 1

    ev.append((-1, 0, "copy", 0, 0))
    for g in range(NBUF - 1):
        copy_stage(-1, g)
    ev.append((-1, 1, "seed", 0, None))
    s = 0

    def stage(seed2=None, seedn=None, base2=None, basen=None):
        nonlocal s
        copy_stage(s, s + NBUF - 1)
        if seed2 is not None:
            ev.append((s, 0, "seed", seed2, None))
        if base2 is not None:
            ev.append((s, 0, "base", base2, None))
        if seedn is not None:
            ev.append((s, 1, "seed", seedn, None))
        if basen is not None:
            ev.append((s, 1, "base", basen, None))
        s += 1

    b = (lambda c: c) if base else (lambda c: None)
    if not ODD:
        for c in range(n_chunks):
            for _ in range(P - 1):
                stage()
            stage(seedn=c + 1 if c + 1 < n_chunks else None, base2=b(c))
    else:
        for c in range(0, n_chunks, 2):
            for q in range(NT):
                if q == NT // 2:
                    stage(seed2=c + 1)
                elif q == NT - 1:
                    stage(seedn=c + 2 if c + 2 < n_chunks else None, base2=b(c + 1))
                elif q == NT // 2 - 1:
                    stage(basen=b(c))
                else:
                    stage()
    assert s == S
    return ev


@pytest.mark.parametrize("NT,n_tp", [(9, 9), (0, 6), (0, 8), (0, 10), (8, 8), (0, 4)])
@pytest.mark.parametrize("n_chunks", [2, 4, 48])
def test_f_rega_chunk_buffers_published_before_read_and_free_before_refill(NT, n_tp, n_chunks):
    """Chunk x's z (and silu(x)) lives in LDS buffer x & 1. Every read of it (seed, base feature)
    must follow the barrier that publishes its copy (barrier g - 1 for a copy issued by
    copy_stage(g), whose group the wait before that barrier completes), and the copy of chunk
    x + 2 into the same buffer must be issued after a barrier that follows every read of chunk x.
    The base variant is exempt at n_tp = 4 (the kernel rejects it there), which this test shows
    is needed."""
    base = n_tp != 4
    ev = f_rega_schedule(NT, n_tp, n_chunks, base=base)
    issue = {x: (stg, g) for (stg, half, kind, x, g) in ev if kind == "copy"}
    for x in range(n_chunks):
        assert x in issue, f"chunk {x} never copied"
    reads = {}
    for (stg, half, kind, x, _) in ev:
        if kind in ("seed", "base"):
            reads.setdefault(x, []).append((stg, half))
    for x, rs in reads.items():
        # the copy riding with group g is complete at barrier g - 1 (chunk 0: the prologue's)
        pub = -1 if x == 0 else issue[x][1] - 1
        for (stg, half) in rs:
            assert (stg, half) > (pub, 0), f"chunk {x} read at {(stg, half)} before barrier {pub}"
        if x + 2 in issue:
            last = max(rs)
            # a barrier between the last read and the refill: a first-half read is followed by
            # barrier stg; a second-half read needs barrier stg + 1
            need = last[0] + 1 if last[1] == 0 else last[0] + 2
            assert issue[x + 2][0] >= need, f"chunk {x + 2} overwrites chunk {x} (read {last}, copy {issue[x + 2]})"
    n_base = sum(1 for e in ev if e[2] == "base")
    assert n_base == (n_chunks if base else 0)


def test_f_rega_base_at_four_features_would_race():
    """The reason the base variant needs chunks of at least 6 features (even counts): at 4, chunk
    x + 2's copy is issued in the stage of chunk x's base read."""
    ev = f_rega_schedule(0, 4, 4, base=True)
    issue = {x: stg for (stg, half, kind, x, g) in ev if kind == "copy"}
    base_reads = {x: stg for (stg, half, kind, x, g) in ev if kind == "base"}
    assert any(issue.get(x + 2, 1 << 30) <= base_reads[x] for x in base_reads)
