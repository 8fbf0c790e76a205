"""Buffer-load offsets of the HIP kernels, modelled on the CPU.

gfx9-family raw buffer loads range-check only the per-lane VGPR offset
(plus the instruction's immediate offset) against the descriptor's
num_records; the scalar offset is added after the check.  A load whose VGPR
offset is in range therefore touches memory at base + voffset + soffset,
and that must lie inside the allocation even though the hardware does not
check the soffset part.  A load whose VGPR offset is out of range returns
zeros and touches nothing.

For every buffer load of the kernels that take one, and for the launch
shapes the library's dispatch gives them, these tests enumerate each lane's
(voffset, soffset) pairs from the kernel's own index arithmetic (cited by
file and line) and assert:
  * every performed load (voffset < num_records) ends inside the
    allocation: voffset + soffset + width <= allocation bytes;
  * every performed load of row-structured data stays inside its own row
    (it reads the row the lane owns, not the next one);
  * rows past the end of the matrix (or of X) are never performed loads.
Kernel constants are read from the headers, so a change there is seen here.
"""
import os
import re

import numpy as np
import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "prism-engine_amd", "csrc")


def _const(header: str, name: str) -> int:
    with open(os.path.join(CSRC, header)) as f:
        text = f.read()
    m = re.search(r"constexpr int " + name + r"\s*=\s*([^;]+);", text)
    assert m, f"{name} not found in {header}"
    expr = m.group(1)
    # resolve references to other constants of the same header
    for ref in re.findall(r"[A-Za-z_]\w*", expr):
        if ref != name:
            expr = expr.replace(ref, str(_const(header, ref)))
    return int(eval(expr, {"__builtins__": {}}))


GW4_BN = _const("gemm_kernels.hpp", "GW4_BN")
GW4_BK = _const("gemm_kernels.hpp", "GW4_BK")
GI_MAX = _const("gemv_kernels.hpp", "kGiMaxRows")
GI_CHUNK = _const("gemv_kernels.hpp", "kGiChunk")
GM_TILES = _const("gemv_mfma.hpp", "kGmTiles")
GM_ROWS = _const("gemv_mfma.hpp", "kGmRows")
GM_WAVES = _const("gemv_mfma.hpp", "kGmWaves")
GM_GROUP = _const("gemv_mfma.hpp", "kGmGroup")


def gi_rows(N, K, num_cu=256, bits=4):
    """The library's layout rule (prism_hip.hip gi_rows)."""
    if K < 2048 or K % (64 if bits == 4 else 512):
        return 0
    G = (-(-N // num_cu) + 7) // 8 * 8
    if bits == 4 and G > GI_MAX and -(-N // 64) <= 2 * num_cu:
        G = 32
    return G if 32 <= G <= GI_MAX else 0


def gi_group_bytes(G, K, bits=4):
    return G * (2 << bits) + G * (K * bits // 8)


def gi_bytes(G, N, K, bits=4):
    return -(-N // G) * gi_group_bytes(G, K, bits)


def gi_chunk_offset(G, r, c, K, bits=4):
    return (r // G) * gi_group_bytes(G, K, bits) + G * (2 << bits) + (c * G + r % G) * GI_CHUNK


def _check(voff, soff, width, num_records, alloc, what):
    voff = np.asarray(voff, dtype=np.int64)
    soff = np.broadcast_to(np.asarray(soff, dtype=np.int64), voff.shape)
    performed = voff < num_records
    end = voff + soff + width
    bad = performed & (end > alloc)
    assert not bad.any(), f"{what}: {int(bad.sum())} loads end past the {alloc}-byte allocation " \
                          f"(first voff {int(voff[bad][0])}, soff {int(soff[bad][0])})"
    return performed


# ---- k_gemm_w4 (gemm_kernels.hpp:470-503): X and index DMA of every block
def _tiles(mt, nt):
    """Every tile of a small grid; for a large one the tiles of the first and
    last M and N blocks (where the ends of X and W are) and a few others."""
    if mt * nt <= 64:
        return range(mt * nt)
    keep = {m * nt + n for m in (0, mt - 1) for n in range(nt)} | {m * nt + n for m in range(mt) for n in (0, nt - 1)}
    keep |= set(np.random.default_rng(0).integers(0, mt * nt, 16).tolist())
    return sorted(keep)


def _gemm_w4(M, N, K, MI, GI):
    G = gi_rows(N, K) if GI else 0
    assert not GI or G, "shape is not a GI shape"
    BM, BN, BK = 32 * MI, GW4_BN, GW4_BK
    XR = 8 * MI
    lane = np.arange(64)[:, None]
    lr8, lc = lane >> 3, (lane & 7) ^ (lane >> 3)
    row_bytes = K // 2
    its = np.arange(K // BK)[None, :]  # K steps (the scalar offset)
    mt, nt = -(-M // BM), -(-N // BN)
    x_alloc = M * K * 2
    w_alloc = gi_bytes(G, N, K) if GI else N * row_bytes
    for t in _tiles(mt, nt):
        n0, m0 = (t % nt) * BN, (t // nt) * BM
        live = min(M - m0, BM)
        x_base = m0 * K * 2  # the descriptor's base is X + m0 * K
        for wave in range(4):
            xv0 = (XR * wave + lr8) * K * 2 + 16 * lc
            for i in range(MI):
                xv = ((xv0 ^ 16) if (i & 1) else xv0) + i * 16 * K
                row = XR * wave + lr8 + 8 * i  # row of the block this lane's DMA reads
                xvb, soff = np.broadcast_arrays(xv, its * 128)
                perf = _check(xvb, soff, 16, live * K * 2, x_alloc - x_base, f"gemm_w4 X M={M} t={t}")
                rowb = np.broadcast_to(row, xvb.shape)
                assert not (perf & (rowb >= live)).any(), "a row past M is read"
                ok = (xvb + soff + 16 <= (rowb + 1) * K * 2) & (xvb + soff >= rowb * K * 2)
                assert ok[perf].all(), "an X load leaves its row"
            if GI:
                # gemm_kernels.hpp:526-530: row 64 w + l, chunk i; rows past N past the range
                grow = n0 + 64 * wave + lane
                wv0 = np.where(grow < N, gi_chunk_offset(G, grow, 0, K), 0x80000000)
                wvs = [wv0, wv0 + G * GI_CHUNK]
                grp_end = (grow // G + 1) * gi_group_bytes(G, K)
            else:
                rows = n0 + 64 * wave + (lane >> 1)
                wv0 = rows * row_bytes + 16 * (lane & 1)
                wvs = [wv0, wv0 + 32 * row_bytes]
            for i, wv in enumerate(wvs):
                wvb, soff = np.broadcast_arrays(wv, its * (2 * G * GI_CHUNK if GI else 32))
                perf = _check(wvb, soff, 16, w_alloc, w_alloc, f"gemm_w4 W N={N} t={t} GI={GI}")
                if GI:
                    assert (wvb + soff + 16 <= np.broadcast_to(grp_end, wvb.shape))[perf].all(), \
                        "a GI load leaves its group"
                else:
                    r = np.broadcast_to(rows + 32 * i, wvb.shape)
                    assert not (perf & (r >= N)).any(), "a weight row past N is read"
                    assert (wvb + soff + 16 <= (r + 1) * row_bytes)[perf].all(), "an index load leaves its row"


@pytest.mark.parametrize("M,N,K,MI,GI", [
    (2048, 14336, 4096, 8, False), (2048, 14336, 4096, 8, True),
    (300, 9100, 2048, 4, True), (64, 8192, 2048, 4, True), (200, 16384, 2048, 8, True), (200, 2000, 2048, 8, False), (96, 2000, 2048, 4, False),
    (33, 4864, 896, 2, False), (600, 4096, 1024, 8, False), (65, 4099, 1024, 2, False),
])
def test_gemm_w4_offsets(M, N, K, MI, GI):
    _gemm_w4(M, N, K, MI, GI)


# ---- k_gemv_mfma (gemv_mfma.hpp:75-110): x rows and index groups
@pytest.mark.parametrize("N,K,nb,bits,GI", [
    (14336, 4096, 8, 4, True), (14336, 4096, 16, 4, False), (14336, 4096, 5, 8, False),
    (4099, 1024, 3, 4, False), (9100, 2048, 16, 4, True), (1000, 384, 4, 8, False),
    (14336, 4096, 16, 8, True), (9100, 2048, 9, 8, True), (8192, 2560, 5, 8, True),
])
def test_gemv_mfma_offsets(N, K, nb, bits, GI):
    lane = np.arange(64)
    n, kq = lane & 15, lane >> 4
    IB = 32 * bits // 8
    ng = K // GM_GROUP
    x_alloc = nb * K * 2
    G = gi_rows(N, K, bits=bits) if GI else 0
    assert not GI or G
    wbytes = gi_bytes(G, N, K, bits) if GI else N * (K * bits // 8)
    row_b = K * bits // 8
    for blk in range(-(-N // GM_ROWS)):
        n0 = blk * GM_ROWS
        for wave in range(GM_WAVES):
            mine = (ng - wave + GM_WAVES - 1) // GM_WAVES if ng > wave else 0
            for g in range(mine):
                k0 = (wave + GM_WAVES * g) * GM_GROUP
                xv = n * K * 2 + kq * 64
                for j in range(4):
                    perf = _check(xv + 16 * j, k0 * 2, 16, x_alloc, x_alloc, "gemv_mfma x")
                    assert ((xv + 16 * j + k0 * 2 + 16) <= (n + 1) * K * 2)[perf].all(), "x load leaves its row"
                    assert not (perf & (n >= nb)).any()
                for t in range(GM_TILES):
                    r = np.minimum(n0 + 16 * t + n, N - 1)
                    if GI:
                        # gemv_mfma.hpp:92,107-108: chunk kq * IB / 16 (+ j), G * 16 bytes apart
                        iv = gi_chunk_offset(G, r, kq * (IB // 16), K, bits)
                        soff = k0 * bits // 8 * G
                        step = G * 16
                        end = (r // G + 1) * gi_group_bytes(G, K, bits)
                    else:
                        iv = r * row_b + kq * IB
                        soff = k0 * bits // 8
                        step = 16
                        end = (r + 1) * row_b
                    for j in range(IB // 16):
                        perf = _check(iv + step * j, soff, 16, wbytes, wbytes, "gemv_mfma index")
                        assert ((iv + step * j + soff + 16) <= end)[perf].all(), "index load leaves its row/group"
                        if GI:  # the chunk is the lane's own row's chunk k0 / 16 + 2 kq + j of the row
                            c = (iv + step * j + soff - (r // G) * gi_group_bytes(G, K, bits) - G * (2 << bits)) // 16
                            assert (c % G == r % G).all() and (c // G == k0 * bits // 128 + kq * (IB // 16) + j).all()


# ---- k_gemv_tile (gemv_tile.hpp:229-262) and k_gemv_lpr (gemv_lpr.hpp:120-135):
# every offset is in the VGPR part; a performed load must end inside the
# allocation (the range check is per load, so alignment matters)
@pytest.mark.parametrize("N,K,bits", [(14336, 4096, 4), (4864, 896, 4), (151936, 896, 4), (3, 1024, 4),
                                      (14336, 4096, 8), (31, 48, 8), (100, 2080, 4)])
def test_gemv_tile_offsets_are_aligned(N, K, bits):
    # x: 16-byte loads at (tid + T t) * 16 against K * 2 bytes
    units = np.arange(0, (K // 8) + 64)
    _check(units * 16, 0, 16, K * 2, K * 2, "gemv_tile x")
    # index: IW dwords per unit, rows clamped to N - 1
    IW = 1 if bits == 4 else 2
    row_dw = K * bits // 32
    for rc in (0, N - 1):
        vo = rc * row_dw * 4 + units * 4 * IW
        perf = _check(vo, 0, 4 * IW, N * row_dw * 4, N * row_dw * 4, "gemv_tile index")
        live = units < K // 8
        assert ((vo + 4 * IW) <= (rc + 1) * row_dw * 4)[perf & live].all()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048), (16384, 2048), (8192, 2112)])
def test_gemv_lpr_offsets(N, K):
    """Chunk c of wave w's range, or an offset past the range (0x80000000);
    lanes past G always past the range (gemv_lpr.hpp:100-140)."""
    G = gi_rows(N, K)
    assert G
    NC = K // 32
    lane = np.arange(64)
    nbytes = gi_bytes(G, N, K)
    for S in (8, 16):
        for w in range(S):
            c0, nch = (w * NC) // S, ((w + 1) * NC) // S - (w * NC) // S
            for g in (0, -(-N // G) - 1):
                base = g * gi_group_bytes(G, K)
                lut = np.where(lane < G, base + lane * 32, 0x80000000)
                for off in (0, 16):
                    perf = _check(lut + off, 0, 16, nbytes, nbytes, "gemv_lpr LUT")
                    assert (perf == (lane < G)).all()
                vbase = np.where(lane < G, base + G * 32 + (c0 * G + lane) * GI_CHUNK, 0x80000000)
                for i in range(nch + 8):  # the ring issues up to P loads past the range
                    vo = vbase + i * G * GI_CHUNK if i < nch else np.full(64, 0x80000000)
                    perf = _check(vo, 0, 16, nbytes, nbytes, "gemv_lpr chunk")
                    assert (perf == ((lane < G) & (i < nch))).all()
                    assert ((vo + 16) <= base + gi_group_bytes(G, K))[perf].all()


@pytest.mark.parametrize("N,K", [(18944, 3584), (16416, 2048), (32768, 4096), (16416, 2560)])
@pytest.mark.parametrize("NM", [1, 2])
def test_gemv_lpr_hg_offsets(N, K, NM):
    """k_gemv_lpr_hg (gemv_lpr.hpp, HG): 32-row groups, lanes 0..31 and
    32..63 in two groups.  NM = 1: groups 2b and 2b + 1 of one matrix under
    one buffer descriptor (one past the last group reads nothing); NM = 2:
    group b of the gate matrix (lanes 0..31) and of the up matrix (lanes
    32..63) through per-lane global loads, so every load the kernel issues
    (a chunk past the wave's range re-reads the lane's first chunk) must be
    inside the lane's own matrix, group and row."""
    G = gi_rows(N, K)
    assert G == 32
    S, NC = 8, K // 32
    gb = gi_group_bytes(G, K)
    groups = -(-N // G)
    nbytes = groups * gb
    assert nbytes == gi_bytes(G, N, K) and nbytes <= 1 << 31
    lane = np.arange(64)
    h, lr = lane >> 5, lane & 31
    blocks = (0, -(-groups // 2) - 1) if NM == 1 else (0, groups - 1)
    for b in blocks:
        g = 2 * b + h if NM == 1 else np.full(64, b)
        gbase = g * gb
        exists = g < groups
        past = 0x80000000 if NM == 1 else None  # NM = 2: no range check; past the range -> chunk c0
        lut = gbase + lr * 32
        for off in (0, 16):
            vo = lut + off
            if NM == 1:
                perf = _check(vo, 0, 16, nbytes, nbytes, "gemv_lpr_hg LUT")
                assert (perf == exists).all()
            else:
                perf = np.ones(64, dtype=bool)
                assert ((vo >= 0) & (vo + 16 <= nbytes)).all(), "global LUT load outside the matrix"
            assert ((vo + 16) <= gbase + (lr + 1) * 32)[perf].all(), "LUT load leaves its row"
        for w in range(S):
            c0, nch = (w * NC) // S, ((w + 1) * NC) // S - (w * NC) // S
            vbase = gbase + G * 32 + (c0 * G + lr) * GI_CHUNK
            for i in range(nch + 8):
                if i < nch:
                    vo = vbase + i * G * GI_CHUNK
                else:
                    vo = np.full(64, past) if NM == 1 else vbase
                if NM == 1:
                    perf = _check(vo, 0, 16, nbytes, nbytes, "gemv_lpr_hg chunk")
                    assert (perf == (exists & (i < nch))).all()
                else:
                    perf = np.ones(64, dtype=bool)
                    assert ((vo >= 0) & (vo + 16 <= nbytes)).all(), "global chunk load outside the matrix"
                assert ((vo >= gbase) & ((vo + 16) <= gbase + gb))[perf].all(), "chunk load leaves its group"
                q = (vo - gbase - G * 32) // GI_CHUNK
                c_is = np.where(i < nch, c0 + i, c0)  # the re-read past the range is chunk c0
                assert ((q % G == lr) & (q // G == c_is))[perf].all()


@pytest.mark.parametrize("N,K", [(14336, 4096), (9100, 2048), (16384, 2048), (8192, 2560)])
def test_gemv_lpr8_offsets(N, K):
    """k_gemv_lpr8 (gemv_lpr.hpp): each wave's 64-byte slice of the lane's
    LUT, then chunk c of its range or an offset past the range; lanes past G
    always past the range; nothing in the scalar offset."""
    G = gi_rows(N, K, bits=8)
    assert G
    S, NC = 8, K // 16
    nch = NC // S
    lane = np.arange(64)
    ngroups = -(-N // G)
    nbytes = ngroups * gi_group_bytes(G, K, 8)  # gridDim.x * gbytes
    assert nbytes == gi_bytes(G, N, K, 8)
    for w in range(S):
        c0 = w * nch
        for g in (0, ngroups - 1):
            base = g * gi_group_bytes(G, K, 8)
            lo = np.where(lane < G, base + lane * 512 + w * 64, 0x80000000)
            for i in range(4):
                perf = _check(lo + 16 * i, 0, 16, nbytes, nbytes, "gemv_lpr8 LUT")
                assert (perf == (lane < G)).all()
                assert ((lo + 16 * i + 16) <= base + (lane + 1) * 512)[perf].all(), "LUT load leaves its row"
            vbase = np.where(lane < G, base + G * 512 + (c0 * G + lane) * GI_CHUNK, 0x80000000)
            for i in range(nch + 8):  # the ring issues loads past the range
                vo = vbase + i * G * GI_CHUNK if i < nch else np.full(64, 0x80000000)
                perf = _check(vo, 0, 16, nbytes, nbytes, "gemv_lpr8 chunk")
                assert (perf == ((lane < G) & (i < nch))).all()
                assert ((vo + 16) <= base + gi_group_bytes(G, K, 8))[perf].all()


LPR8M_AHEAD = _const("gemv_lpr_args.hpp", "kLpr8mAhead")
LPR8M_XDW = _const("gemv_lpr_args.hpp", "kLpr8mXDw")
LPR8M_XPAD = _const("gemv_lpr_args.hpp", "kLpr8mXPad")


@pytest.mark.parametrize("N,K,nb", [(14336, 4096, 8), (14336, 4096, 5), (9100, 2048, 8), (16384, 2048, 5),
                                    (8192, 2560, 8), (8192, 2560, 6), (9000, 4608, 7), (9000, 6144, 5),
                                    (12000, 2048, 6)])
def test_gemv_lpr8m_offsets(N, K, nb):
    """k_gemv_lpr8m (gemv_lpr8m.hip): wave w's 64-byte slices of the LUTs of
    rows r and 32 + r; x in 16-byte pieces (eight per thread, past nb*K
    nothing); double step s's chunk c0 + 2s + h of row 32t + r, or an offset
    past the block from nd on (the loop requests AH past the end); and the
    LDS indices of the x reads and the partials."""
    G = gi_rows(N, K, bits=8)
    xrow = K // 2 + LPR8M_XPAD  # LDS dwords per vector
    assert G and nb * xrow <= LPR8M_XDW and nb <= 32, "the host's condition for this kernel"
    assert nb * K // 8 <= 8 * 512, "x pieces: at most eight per thread"
    Q, AH = 4, LPR8M_AHEAD
    nd = K // (Q * 32)
    assert nd % AH == 0, "the loop runs whole blocks of AH double steps"
    lane = np.arange(64)
    r32, h = lane % 32, lane // 32
    ngroups = -(-N // G)
    gb = gi_group_bytes(G, K, 8)
    nbytes = ngroups * gb
    for g in (0, ngroups - 1):
        base = g * gb
        for w in range(8):
            t, q = w & 1, w >> 1
            for rows in (r32, 32 + r32):
                lo = np.where(rows < G, base + rows * 512 + w * 64, 0x80000000)
                for i in range(4):
                    perf = _check(lo + 16 * i, 0, 16, nbytes, nbytes, "gemv_lpr8m LUT")
                    assert (perf == (rows < G)).all()
                    assert ((lo + 16 * i + 16) <= base + (rows + 1) * 512)[perf].all(), "LUT load leaves its row"
            row = 32 * t + r32
            c0 = q * (K // (Q * 16))
            ibase = np.where(row < G, base + G * 512 + ((c0 + h) * G + row) * GI_CHUNK, 0x80000000)
            for s in range(nd + AH):
                io = ibase + s * 2 * G * GI_CHUNK if s < nd else np.full(64, 0x80000000)
                perf = _check(io, 0, 16, nbytes, nbytes, "gemv_lpr8m chunk")
                assert (perf == ((row < G) & (s < nd))).all()
                assert ((io + 16) <= base + gb)[perf].all(), "chunk load leaves its group"
                # chunk c0 + 2s + h stays inside the wave's K quarter
                assert (c0 + 2 * s + h < c0 + K // (Q * 16))[perf].all()
            # x from LDS: lanes r < nb read dwords xoff + 16 s .. + 7 of their
            # vector's row (xrow dwords, the last kLpr8mXPad of them padding)
            xoff = r32 * xrow + 8 * (c0 + h)
            live = r32 < nb
            last = xoff + 16 * (nd - 1) + 8
            assert (last[live] <= r32[live] * xrow + K // 2).all()
            # the lanes' x elements are those of their weight bytes
            for s in (0, nd - 1):
                for j in (0, 1):
                    xel = 2 * (xoff + 16 * s - r32 * xrow) + 8 * j
                    wel = 16 * (c0 + 2 * s + h) + 8 * j
                    assert (xel == wel).all()
            # 16 lanes per clock for 16-byte reads: the live lanes of each
            # 16-lane group start in distinct 4-bank groups
            for grp in range(4):
                ln = np.arange(16 * grp, 16 * grp + 16)
                ln = ln[r32[ln] < nb]
                banks = (xoff[ln] % 64) // 4
                assert len(set(banks.tolist())) == len(ln), "x reads conflict"
    tid = np.arange(512)
    xq = nb * K // 8
    for i in range(8):
        p = tid + 512 * i
        perf = _check(np.where(p < xq, p * 16, 0x80000000), 0, 16, nb * K * 2, nb * K * 2, "gemv_lpr8m x")
        assert (perf == (p < xq)).all()
    assert ((tid[:, None] + 512 * np.arange(8)[None, :]) < xq).sum() == xq, "x pieces cover x once"
    p = np.arange(xq)
    dst = (p // (K // 8)) * xrow + 4 * (p % (K // 8))
    assert dst.max() + 4 <= LPR8M_XDW and len(np.unique(dst)) == xq
    # partials: [Q][2][32][33] floats in the x region
    assert (Q * 2 * 32 + 31) * 33 + 31 < LPR8M_XDW


@pytest.mark.parametrize("N,K,nb", [(14336, 4096, 8), (14336, 4096, 3), (9100, 2048, 8), (16384, 2048, 5),
                                    (14336, 8192, 4), (9000, 2304, 7), (12000, 3328, 6)])
def test_gemv_lpr4m_offsets(N, K, nb):
    """k_gemv_lpr4m (gemv_lpr8m.hip): the LUT of row `lane` (two 16-byte
    loads, rows past G an offset past the range); x in 16-byte pieces; double
    step s's chunk c0 + 2s + h of row 32t + r, or an offset past the range
    from nd on (the loop requests AH past its last step, in whole blocks of
    AH even when AH does not divide nd); the x reads' LDS dwords, the table's
    and the lookups' LDS indices."""
    G = gi_rows(N, K)
    xrow = K // 2 + LPR8M_XPAD
    assert G > 32 and K % 256 == 0 and 3 <= nb <= 8 and nb * xrow <= LPR8M_XDW, "the host's condition"
    Q, AH = 4, LPR8M_AHEAD
    nc = K // 32
    nd = nc // (Q * 2)
    lane = np.arange(64)
    r32, h = lane % 32, lane // 32
    ngroups = -(-N // G)
    gb = gi_group_bytes(G, K)
    nbytes = ngroups * gb
    for g in (0, ngroups - 1):
        base = g * gb
        lo = np.where(lane < G, base + lane * 32, 0x80000000)
        for i in range(2):
            perf = _check(lo + 16 * i, 0, 16, nbytes, nbytes, "gemv_lpr4m LUT")
            assert (perf == (lane < G)).all()
            assert ((lo + 16 * i + 16) <= base + G * 32)[perf].all(), "LUT load leaves the group's LUTs"
        for w in range(8):
            t, q = w & 1, w >> 1
            row = 32 * t + r32
            c0 = q * (nc // Q)
            ibase = np.where(row < G, base + G * 32 + ((c0 + h) * G + row) * GI_CHUNK, 0x80000000)
            steps = -(-nd // AH) * AH + AH  # every ld() the loop issues
            for s in range(steps):
                io = ibase + s * 2 * G * GI_CHUNK if s < nd else np.full(64, 0x80000000)
                perf = _check(io, 0, 16, nbytes, nbytes, "gemv_lpr4m chunk")
                assert (perf == ((row < G) & (s < nd))).all()
                assert ((io + 16) <= base + gb)[perf].all(), "chunk load leaves its group"
                assert (c0 + 2 * s + h < c0 + nc // Q)[perf].all(), "chunk outside the wave's K quarter"
            # x from LDS: lanes r < nb read dwords xoff + 32 s + 4 j .. + 3, j < 4
            xoff = r32 * xrow + 16 * (c0 + h)
            live = r32 < nb
            last = xoff + 32 * (nd - 1) + 16
            assert (last[live] <= r32[live] * xrow + K // 2).all()
            for s in (0, nd - 1):
                for j in range(4):
                    xel = 2 * (xoff + 32 * s + 4 * j - r32 * xrow)
                    wel = 32 * (c0 + 2 * s + h) + 8 * j
                    assert (xel == wel).all(), "x and weight elements of an MFMA differ"
            for grp in range(4):
                ln = np.arange(16 * grp, 16 * grp + 16)
                ln = ln[r32[ln] < nb]
                banks = (xoff[ln] % 64) // 4
                assert len(set(banks.tolist())) == len(ln), "x reads conflict"
    # the table: wave w writes entries w + 8i of every row at dword 64 e + row;
    # a lookup of index byte b for row 32t + r reads dword 64 b + row
    e = (np.arange(8)[:, None] + 8 * np.arange(32)[None, :]).ravel()
    assert sorted(e.tolist()) == list(range(256)), "the waves build every entry once"
    assert (e.max() * 64 + 63) < 256 * 64 and 255 * 64 + 63 < 256 * 64
    tid = np.arange(512)
    xq = nb * K // 8
    for i in range(8):
        p = tid + 512 * i
        perf = _check(np.where(p < xq, p * 16, 0x80000000), 0, 16, nb * K * 2, nb * K * 2, "gemv_lpr4m x")
        assert (perf == (p < xq)).all()
    assert ((tid[:, None] + 512 * np.arange(8)[None, :]) < xq).sum() == xq, "x pieces cover x once"


LPR4Q_AHEAD = _const("gemv_lpr_args.hpp", "kLpr4qAhead")
LPR4Q_RING = _const("gemv_lpr_args.hpp", "kLpr4qRing")


@pytest.mark.parametrize("N,K,nb", [(14336, 4096, 4), (14336, 4096, 3), (9100, 2048, 4), (14336, 8192, 4),
                                    (9000, 2304, 3), (12000, 3328, 4)])
def test_gemv_lpr4q_offsets(N, K, nb):
    """k_gemv_lpr4q (gemv_lpr8m.hip): the LUT of row `lane` (two 16-byte
    loads, lanes past G an offset past the range); x in 16-byte pieces; chunk
    c0 + i of row `lane`, or an offset past the range from the wave's chunk
    count on (the compile-time sequence requests up to kLpr4qAhead past it,
    the run-time loop a block of kLpr4qRing); each lane's LDS x reads stay
    inside its vector and hold the k its A operand holds."""
    G = gi_rows(N, K)
    xrow = K // 2 + LPR8M_XPAD
    assert G > 32 and K % 256 == 0 and nb in (3, 4) and nb * xrow <= LPR8M_XDW, "the host's condition"
    S = 8
    nc = K // 32
    nch = nc // S
    compile_time = nch in (8, 16)
    ahead = LPR4Q_AHEAD if compile_time else LPR4Q_RING
    lane = np.arange(64)
    ngroups = -(-N // G)
    gb = gi_group_bytes(G, K)
    nbytes = ngroups * gb
    for g in (0, ngroups - 1):
        base = g * gb
        lo = np.where(lane < G, base + lane * 32, 0x80000000)
        for i in range(2):
            perf = _check(lo + 16 * i, 0, 16, nbytes, nbytes, "gemv_lpr4q LUT")
            assert (perf == (lane < G)).all()
            assert ((lo + 16 * i + 16) <= base + G * 32)[perf].all(), "LUT load leaves the group's LUTs"
        for w in range(S):
            c0 = (w * nc) // S
            assert ((w + 1) * nc) // S - c0 == nch
            vbase = np.where(lane < G, base + G * 32 + (c0 * G + lane) * GI_CHUNK, 0x80000000)
            for i in range(nch + ahead):  # every chunk request, the ones past the range included
                vo = vbase + i * G * GI_CHUNK if i < nch else np.full(64, 0x80000000)
                perf = _check(vo, 0, 16, nbytes, nbytes, "gemv_lpr4q chunk")
                assert (perf == ((lane < G) & (i < nch))).all()
                assert ((vo + 16) <= base + gb)[perf].all(), "chunk load leaves its group"
            # LDS x reads of lane l: vector min(l % 4, nb - 1), bytes 64 (c0 + c) + 16 m, m < 4
            vec = np.minimum(lane % 4, nb - 1)
            for c in (0, nch - 1):
                for m in range(4):
                    off = vec * xrow * 4 + (c0 + c) * 64 + 16 * m
                    assert ((off + 16) <= vec * xrow * 4 + K * 2).all(), "x read leaves its vector"
                    for half in range(2):  # MFMA step 2 m + half: x elements and weight elements agree
                        step = 2 * m + half
                        xel = (off + 8 * half - vec * xrow * 4) // 2
                        assert (xel == 32 * (c0 + c) + 4 * step).all()
    tid = np.arange(512)
    xq = nb * K // 8
    for i in range(8):
        p = tid + 512 * i
        perf = _check(np.where(p < xq, p * 16, 0x80000000), 0, 16, nb * K * 2, nb * K * 2, "gemv_lpr4q x")
        assert (perf == (p < xq)).all()
        b, o = p // (K // 8), p % (K // 8)
        assert ((b * xrow + 4 * o + 4) <= LPR8M_XDW)[p < xq].all(), "x store leaves its LDS region"
    assert ((tid[:, None] + 512 * np.arange(8)[None, :]) < xq).sum() == xq, "x pieces cover x once"
