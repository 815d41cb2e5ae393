"""Generates the tile loop of ``bwd_dq_wide_kernel`` as gfx950 assembly.

The arithmetic is the dQ part of the derivative of the reference branch
kernel (swiattn_gqa_prefill_varlen.py V:176-241; the reference itself is
forward-only, V:14-15): for each routed row r and legal key j of its range,
P = 2^(c q_r.k_j - LSE_r) with the forward's log2 LSE, dS = P (dO_r.v_j -
Delta_r) rounded to bf16, dq_r = scale * sum_j dS k_j.  Keys outside a row's
range get S = -inf, hence P = 0 and dS = 0.

Layout.  A work item is 256 rows (eight 32-row blocks of the backward's row
info), 64 per wave, one wave per SIMD, and the keys of its range in 64-key
tiles.  Per lane that takes the dQ^T accumulators (128 fp32), the Q^T and
dO^T operands (64 registers each), two score tiles for the software
pipeline (128), the dP^T tile (64) and the operand staging: the dQ^T
accumulators and the Q^T / dO^T operands fill the 256 AGPRs (the matrix
cores read and accumulate there directly), S, dP and everything else the
256 VGPRs.  Three products per tile, all in the transposed form so that
the accumulators of one are the B operands of the next:

  S^T  = K Q^T      (A: K rows from LDS, B: Q^T in AGPRs)
  D    = V dO^T - Delta  (A: V rows from LDS, B: dO^T in AGPRs, starting
                     from -Delta of each row, moved in before the MFMAs)
  dQ^T += K^T dS^T  (A: K^T by transposing LDS reads of the same K tile,
                     B: dS^T packed to bf16 from the S accumulators)

The packed dS^T of a tile is written back over the first 32 registers of
its own S buffer, and the transposing reads deliver the keys of each
16-key group in the order one lane holds them, so no data moves between
lanes.

Step r (phase q = r mod 4, tile r's S in buffer r mod 2) issues 96 MFMAs:
dQ^T(r) for keys 0-15, S^T(r+1) (keys 0-31, then 32-63), dQ^T(r) keys
16-31, dP^T(r+1) keys 0-31, dQ^T(r) keys 32-63, dP^T(r+1) keys 32-63, so
that the scores of tile r+1 are complete early and their exponentials can
spread over the rest of the step.  Its VALU work: dS of tile r's keys 32-63
and their packing (before the dQ^T MFMAs that read them), P = 2^(S c -
LSE) of tile r+1 (after the masking of tile r+1 when it lies outside the
range every row of the wave covers), dS = P D (one multiply per element) of
tile r+1's keys 0-31 and their packing, and the -Delta starting values of
the dP^T accumulators of tile r+1.  A list scheduler spreads it over the MFMA slots, at most one
exponential and one instruction feeding an exponential per slot.  K and V tiles stream through four-slot LDS rings, staged by the
four waves with global -> LDS loads three (K) and four (V) steps ahead;
the loop is unrolled four steps so that every LDS address is a base
register plus an immediate offset.

Register map (per lane; "rb" = 32-row block of the wave's 64 rows, "h" =
32-key half of a tile, "db" = 32-wide block of head_dim):
  a[0:127]    dQ^T accumulators, (db, rb) at 32 db + 16 rb
  a[128:191]  Q^T operands, k-step kk, rb at 128 + 8 kk + 4 rb
  a[192:255]  dO^T operands, likewise
  v[0:63], v[64:127]  S tiles (ping-pong), (rb, h) at +32 rb + 16 h; after
              the packing, dS^T operand (k-step s2, rb) at +8 s2 + 4 rb
  v[128:191]  dP^T - Delta tile, same layout
  v[192:207]  four operand staging sets
  v[208:255]  LDS addresses, row state, mask temporaries, DMA and store
              offsets; (-Delta, -Delta) of row block 0 at 234-235 and of
              row block 1 at 254-255
"""

from __future__ import annotations

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import gen_fwd_wide as F  # noqa: E402
from gen_fwd_wide import (Block, Ins, areg, branch, half_elems, insert_waits, label, mfma,  # noqa: E402
                          pad_program, regs, s_in, salu, schedule, sreg, valu, vreg, waitcnt)

# ---------------------------------------------------------------------------
# registers
# ---------------------------------------------------------------------------
DQ_A, Q_A, DO_A = 0, 128, 192
S_V = (0, 64)
D_V = 128
ST_V, N_SETS = 192, 4        # operand staging sets (4 registers each)
LEAD = 3                     # operands read ahead of the MFMA pair that takes them
KOFF_V = 208                 # [kk] K row read address (ring slot 0)
VOFF_V = 216                 # [kk] V row read address (ring slot 0)
TOFF_V = 224                 # [db][a] transposing read address (ring slot 0, k-step 0)
V_NLSE = 232                 # [rb] -LSE
V_DLT = 234                  # [rb] Delta (the prologue turns 234-235 into V_NDLT[0])
V_KSR = 236                  # [rb] row start - 4 hh
V_SPAN = 238                 # [rb] row key count
V_LO = 240                   # [rb] mask: row start - 4 hh - first key of the tile
V_MK = 242                   # 242..245 mask temporaries
V_NINF = 246
V_TMP = 247
V_KDMA = 248                 # [i] global offsets of this lane's K / V DMA loads
V_DQOFF = 252                # [rb] dq row byte offset (+ 8 hh); 254, 255: Q row offsets (prologue)
V_QOFF = 254
V_NDLT = (234, 254)          # [rb] (-Delta, -Delta) register pairs, the loop's dP^T starting values

S_T0, S_T1 = 52, 53
S_R1 = 54                    # r + 1 for step r (the tile whose S and dP the step computes)
S_N = 55                     # tile count
S_SPAN = 56                  # it1 - it0
S_KEY0 = 57                  # first key of tile r + 1 (masked steps)
S_KBYTES, S_VBYTES = 58, 59  # bytes from the current K / V descriptor base to the item's end
S_KRS, S_VRS = 60, 64        # K / V buffer descriptors
S_PAIRS = (68, 70, 72, 74)   # VALU compare results
S_FIRST, S_LASTC = 52, 75

NEG_INF_BITS = 0xFF800000
RSRC_WORD3 = F.RSRC_WORD3
TILE_BYTES = 16384
SLOTS = 4
V_RING = SLOTS * TILE_BYTES
LDS_BYTES = 2 * V_RING
# Per-lane inputs written by the C++ part: seven groups of four words per
# lane, 1 KiB per group and wave; waves 0-1 in K slot 3, waves 2-3 in V slot
# 3 (slots the prologue does not stage into).
AUX_GROUPS = 7
# Per-wave staging of the dq rows in the epilogue (in K slots 0-2, free
# after the loop): 32 rows at a 272-byte stride, then their byte offsets.
EPI_REGION = 32 * 272 + 128


# ---------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------


def st(o):
    return ST_V + 4 * (o % N_SETS)


def op_reads(op, o, q):
    """LDS reads of operand op (index o in the step) for phase q."""
    kind, a, b = op
    dst = st(o)
    if kind == "k":            # K rows of S^T(r+1): half a, k-step b
        off = ((q + 1) % SLOTS) * TILE_BYTES + a * 8192
        return [Ins(f"ds_read_b128 {vreg(dst, 4)}, {vreg(KOFF_V + b)} offset:{off}", "lds",
                    {f"v{KOFF_V + b}"}, regs("v", dst, 4), lgkm=True)]
    if kind == "v":            # V rows of dP^T(r+1)
        off = ((q + 1) % SLOTS) * TILE_BYTES + a * 8192
        return [Ins(f"ds_read_b128 {vreg(dst, 4)}, {vreg(VOFF_V + b)} offset:{off}", "lds",
                    {f"v{VOFF_V + b}"}, regs("v", dst, 4), lgkm=True)]
    # "t": K^T of dQ^T(r): k-step a (16 keys), head_dim block b; two
    # transposing reads of tile r's K (rows 16 a .. 16 a + 15)
    off = (q % SLOTS) * TILE_BYTES + a * 4096
    out = []
    for half in range(2):
        adr = TOFF_V + 2 * b + half
        out.append(Ins(f"ds_read_b64_tr_b16 {vreg(dst + 2 * half, 2)}, {vreg(adr)} offset:{off}", "lds",
                       {f"v{adr}"}, regs("v", dst + 2 * half, 2), lgkm=True))
    return out


def op_mfmas(op, o, sc, sn):
    kind, a, b = op
    src = ("v", st(o))
    if kind == "k":
        return [mfma(("v", sn + 32 * rb + 16 * a), src, ("a", Q_A + 8 * b + 4 * rb), b > 0) for rb in range(2)]
    if kind == "v":
        # accumulates onto -Delta (prefill): the result is dP^T - Delta
        return [mfma(("v", D_V + 32 * rb + 16 * a), src, ("a", DO_A + 8 * b + 4 * rb), True) for rb in range(2)]
    return [mfma(("a", DQ_A + 32 * b + 16 * rb), src, ("v", sc + 8 * a + 4 * rb), True) for rb in range(2)]


def ops_of(kind):
    gq = lambda s2s: [("t", s2, db) for s2 in s2s for db in range(4)]  # noqa: E731
    gs = lambda h: [("k", h, kk) for kk in range(8)]                    # noqa: E731
    gd = lambda h: [("v", h, kk) for kk in range(8)]                    # noqa: E731
    if kind == "pre":
        return gs(0) + gd(0) + gs(1) + gd(1)
    if kind == "last":
        return gq((0, 1, 2, 3))
    return gq((0,)) + gs(0) + gs(1) + gq((1,)) + gd(0) + gq((2, 3)) + gd(1)


NEXT_OPS = [("t", 0, db) for db in range(LEAD)]    # read before the next step's barrier
N_PRE_LDS = 2 * LEAD


def dma(kind, i, slot):
    rs = S_KRS if kind == "k" else S_VRS
    base = slot * TILE_BYTES + (0 if kind == "k" else V_RING) + i * 1024
    return [salu(f"s_add_u32 m0, {s_in('ldsw')}, {base}", wr={"m0"}),
            Ins(f"buffer_load_dwordx4 {vreg(V_KDMA + i)}, {sreg(rs, 4)}, 0 offen lds", "dma",
                regs("s", rs, 4) | {"m0", f"v{V_KDMA + i}"}, set(), vm=True)]


def desc_advance(kind):
    """Next tile: base += tile, the bytes left to the item's end shrink by a
    tile, and the record count is what is left (none past the item's last
    tile, part of the keys' last tile)."""
    rs, nb = (S_KRS, S_KBYTES) if kind == "k" else (S_VRS, S_VBYTES)
    step = s_in("ktilebytes")
    return [salu(f"s_add_u32 {sreg(rs)}, {sreg(rs)}, {step}"),
            salu(f"s_addc_u32 {sreg(rs + 1)}, {sreg(rs + 1)}, 0"),
            salu(f"s_sub_i32 {sreg(nb)}, {sreg(nb)}, {step}"),
            salu(f"s_max_i32 {sreg(rs + 2)}, {sreg(nb)}, 0")]


def exps(s, h):
    """P = 2^(s c - LSE) in place for half h of the S tile at s."""
    out = []
    for rb, x in half_elems(s, h):
        out.append(valu(f"v_fma_f32 {vreg(x)}, {vreg(x)}, {s_in('c')}, {vreg(V_NLSE + rb)}",
                        {f"v{x}", f"v{V_NLSE + rb}"}, {f"v{x}"}))
        out[-1].feeds_trans = True
        out.append(valu(f"v_exp_f32 {vreg(x)}, {vreg(x)}", {f"v{x}"}, {f"v{x}"}, trans=True))
    return out


def prefill(h):
    """The dP^T accumulators of half h start from -Delta of their row (eight
    64-bit moves per row block from its (-Delta, -Delta) pair), so that the
    MFMAs leave dP^T - Delta there."""
    out = []
    for rb in range(2):
        base = D_V + 32 * rb + 16 * h
        pr = V_NDLT[rb]
        for i in range(0, 16, 2):
            out.append(valu(f"v_mov_b64 {vreg(base + i, 2)}, {vreg(pr, 2)}", {f"v{pr}", f"v{pr + 1}"},
                            {f"v{base + i}", f"v{base + i + 1}"}))
    return out


def dss(s, h):
    """dS = P (dP - Delta) in place for half h (dP - Delta is what the dP^T
    MFMAs left in D)."""
    out = []
    for rb, x in half_elems(s, h):
        d = D_V + (x - s)
        out.append(valu(f"v_mul_f32 {vreg(x)}, {vreg(x)}, {vreg(d)}", {f"v{x}", f"v{d}"}, {f"v{x}"}))
    return out


def packs(s, h):
    """dS^T operands of half h packed to bf16 over the row block 0 half h
    registers: k-step s2 = 2 h + (i >= 8), register (i % 8) / 2 holds
    elements i, i+1 of the row block.  Row block 0 is packed first: row
    block 1's operands land on row block 0's elements 4-7 and 12-15."""
    out = []
    for rb in range(2):
        for i in range(0, 16, 2):
            base = s + 32 * rb + 16 * h
            d = s + 8 * (2 * h + (i >= 8)) + 4 * rb + (i % 8) // 2
            out.append(valu(f"v_cvt_pk_bf16_f32 {vreg(d)}, {vreg(base + i)}, {vreg(base + i + 1)}",
                            {f"v{base + i}", f"v{base + i + 1}"}, {f"v{d}"}))
    return out


def mask(s, h):
    """Scores of half h outside each row's [start, end) set to -inf.
    Register r of the half is key 32 h + 8 (r >> 2) + 4 hh + (r & 3) of the
    tile; the row bounds were shifted by 4 hh, so it is legal iff
    (off - lo) < span, unsigned, with lo = start - 4 hh - key0."""
    out = []
    for rb in range(2):
        out.append(valu(f"v_subrev_u32 {vreg(V_LO + rb)}, {sreg(S_KEY0)}, {vreg(V_KSR + rb)}",
                        {f"v{V_KSR + rb}", f"s{S_KEY0}"}, {f"v{V_LO + rb}"}))
    elems = [(rb, r) for rb in range(2) for r in range(16)]
    for g in range(0, len(elems), 4):
        grp = elems[g:g + 4]
        for k, (rb, r) in enumerate(grp):
            off = 32 * h + 8 * (r >> 2) + (r & 3)
            out.append(valu(f"v_sub_u32 {vreg(V_MK + k)}, {off}, {vreg(V_LO + rb)}", {f"v{V_LO + rb}"},
                            {f"v{V_MK + k}"}))
        for k, (rb, r) in enumerate(grp):
            p = S_PAIRS[k]
            out.append(valu(f"v_cmp_gt_u32_e64 {sreg(p, 2)}, {vreg(V_SPAN + rb)}, {vreg(V_MK + k)}",
                            {f"v{V_SPAN + rb}", f"v{V_MK + k}"}, {f"s{p}", f"s{p + 1}"}))
        for k, (rb, r) in enumerate(grp):
            x = s + 32 * rb + 16 * h + r
            p = S_PAIRS[k]
            out.append(valu(f"v_cndmask_b32_e64 {vreg(x)}, {vreg(V_NINF)}, {vreg(x)}, {sreg(p, 2)}",
                            {f"v{x}", f"v{V_NINF}"}, {f"v{x}"}, mask_rd={f"s{p}", f"s{p + 1}"}))
    return out


# ---------------------------------------------------------------------------
# steps
# ---------------------------------------------------------------------------
# Step r (phase q): dQ^T(r) from tile r's K in K slot q, S^T(r+1) and
# dP^T(r+1) from K(r+1) / V(r+1) in slot (q+1) % 4 of each ring.  It stages
# K(r+3) into K slot (q+3) % 4 (tile r-1's, last read by step r-1) and
# V(r+4) into V slot q (tile r's V, last read by step r-1), and at its end
# reads the first K^T operands of step r+1 (tile r+1's K, in LDS since
# step r-1's barrier).

DMA_AT = {"full": (4, 16, 28, 40, 52, 64, 76, 88), "pre": (4, 12, 20, 28, 36, 44, 52, 60)}


def step_code(q, kind, masked):
    """One step's instructions: the scheduled MFMAs with their operand
    reads, DMAs and VALU work."""
    par = q % 2
    sc, sn = S_V[par], S_V[1 - par]     # tile r, tile r + 1
    ops = ops_of(kind)
    mf = []
    for o, op in enumerate(ops):
        mf += op_mfmas(op, o, sc, sn)
    nm = len(mf)
    # operand reads: op o before the MFMA pair of op o - LEAD; the next
    # step's first operands continue the sequence
    reads = {}
    seq = [(o, op, q) for o, op in enumerate(ops)]
    if kind != "last":
        seq += [(len(ops) + o, op, (q + 1) % 4) for o, op in enumerate(NEXT_OPS)]
    first = 0 if kind == "pre" else LEAD
    for o, op, qq in seq:
        if o < first:
            continue
        at = max(0, 2 * (o - LEAD) + 1)
        reads.setdefault(at, []).extend(op_reads(op, o, qq))
    dmas = {}
    if kind != "last":
        ks, vs = (q + 3) % 4, (q if kind == "full" else 3)
        if kind == "pre":
            ks = 2
        at = DMA_AT[kind]
        for i in range(4):
            dmas[at[i]] = dma("k", i, ks) + (desc_advance("k") if i == 3 else [])
            dmas[at[4 + i]] = dma("v", i, vs) + (desc_advance("v") if i == 3 else [])

    def side(i):
        return dmas.get(i, []) + reads.get(i, [])

    carried = []
    if kind != "pre":
        carried = dss(sc, 1) + packs(sc, 1)
    if kind != "last":
        # carried work goes before the first MFMA that touches its
        # registers: here the dP^T MFMAs that accumulate onto it
        carried += prefill(0) + prefill(1)
    vl = list(carried)
    if kind != "last":
        pre_mask = []
        if masked:
            pre_mask = [salu(f"s_lshl_b32 {sreg(S_KEY0)}, {sreg(S_R1)}, 6"),
                        salu(f"s_add_u32 {sreg(S_KEY0)}, {sreg(S_KEY0)}, {s_in('key0')}")]
            if kind == "pre":
                pre_mask = [salu(f"s_mov_b32 {sreg(S_KEY0)}, {s_in('key0')}")]
        vl += pre_mask
        vl += (mask(sn, 0) if masked else []) + exps(sn, 0)
        vl += (mask(sn, 1) if masked else []) + exps(sn, 1)
        vl += dss(sn, 0) + packs(sn, 0)
    lead = 0 if kind == "pre" else 3
    o, _ = schedule(mf, vl, side, carry=False, n_carried=len(carried), lead_cap=lead, one_feed=True)
    return o


def step_blocks(tag, q, kind, end_label):
    u = "%="
    blocks = []
    if kind == "pre":
        blocks.append(Block(f"L{tag}_a_{u}", step_code(q, "pre", True)))
        return blocks
    # DMAs issued two steps ago and earlier have landed in every wave; the
    # eight of the previous step may still be in flight, and so may the
    # previous step's last reads (of tile r's K, which no DMA of this step
    # writes)
    blocks.append(Block(f"L{tag}_s_{u}", [waitcnt(vm=8, lgkm=N_PRE_LDS), Ins("s_barrier", "barrier")]))
    if kind == "last":
        blocks.append(Block(f"L{tag}_a_{u}", step_code(q, "last", False)
                            + [branch("s_branch", end_label, cond=False)]))
        return blocks
    # tile r + 1 needs the range mask iff it lies outside [it0, it1)
    blocks.append(Block(f"L{tag}_mt_{u}", [salu(f"s_sub_u32 {sreg(S_T1)}, {sreg(S_R1)}, {s_in('it0')}"),
                                           salu(f"s_cmp_ge_u32 {sreg(S_T1)}, {sreg(S_SPAN)}"),
                                           branch("s_cbranch_scc1", f"L{tag}_am_{u}")]))
    blocks.append(Block(f"L{tag}_au_{u}", step_code(q, "full", False)
                        + [branch("s_branch", end_label, cond=False)]))
    blocks.append(Block(f"L{tag}_am_{u}", step_code(q, "full", True)))
    return blocks


def prologue():
    """Per-lane inputs from LDS, Q^T and dO^T rows into their AGPRs, dQ^T =
    0, descriptors and constants, K(0), V(0), K(1), V(1), V(2) staged, then
    wait and barrier."""
    # The compiler's code before this block wrote some of the input SGPRs
    # with VALU instructions (v_readfirstlane); a buffer instruction reading
    # such an SGPR needs 5 wait states, which the compiler cannot see inside
    # inline assembly.
    out = [salu("s_mov_b64 exec, -1"), Ins("s_nop 7", "nop")]
    t = V_TMP
    out += [valu(f"v_mbcnt_lo_u32_b32 {vreg(t)}, -1, 0", set(), {f"v{t}"}),
            valu(f"v_mbcnt_hi_u32_b32 {vreg(t)}, -1, {vreg(t)}", {f"v{t}"}, {f"v{t}"}),
            valu(f"v_lshl_add_u32 {vreg(t)}, {vreg(t)}, 4, {s_in('aux')}", {f"v{t}"}, {f"v{t}"})]
    # group -> destination: 0 dq / Q offsets, 1 -LSE / Delta, 2 row bounds,
    # 3-4 transposing read addresses, 5 DMA offsets, 6 K read address (+3 unused)
    dst = {0: V_DQOFF, 1: V_NLSE, 2: V_KSR, 3: TOFF_V, 4: TOFF_V + 4, 5: V_KDMA, 6: D_V}
    for g in range(AUX_GROUPS):
        d = dst[g]
        out.append(Ins(f"ds_read_b128 {vreg(d, 4)}, {vreg(t)} offset:{g * 1024}", "lds", {f"v{t}"},
                       regs("v", d, 4), lgkm=True))
    out += [
        salu(f"s_mov_b32 {sreg(S_N)}, {s_in('ntiles')}"),
        salu(f"s_mov_b64 {sreg(S_KRS, 2)}, {s_in('kbase')}"),
        salu(f"s_mov_b32 {sreg(S_KBYTES)}, {s_in('kbytes')}"),
        salu(f"s_max_i32 {sreg(S_KRS + 2)}, {sreg(S_KBYTES)}, 0"),
        salu(f"s_mov_b32 {sreg(S_KRS + 3)}, {RSRC_WORD3:#x}"),
        salu(f"s_mov_b64 {sreg(S_VRS, 2)}, {s_in('vbase')}"),
        salu(f"s_mov_b32 {sreg(S_VBYTES)}, {s_in('kbytes')}"),
        salu(f"s_max_i32 {sreg(S_VRS + 2)}, {sreg(S_VBYTES)}, 0"),
        salu(f"s_mov_b32 {sreg(S_VRS + 3)}, {RSRC_WORD3:#x}"),
        salu(f"s_sub_i32 {sreg(S_SPAN)}, {s_in('it1')}, {s_in('it0')}"),
        salu(f"s_max_i32 {sreg(S_SPAN)}, {sreg(S_SPAN)}, 0"),
        salu(f"s_mov_b32 {sreg(S_R1)}, 0"),
    ]
    for rb in range(2):
        for kk in range(8):
            d = Q_A + 8 * kk + 4 * rb
            out.append(Ins(f"buffer_load_dwordx4 {areg(d, 4)}, {vreg(V_QOFF + rb)}, {s_in('qrsrc')}, 0 offen "
                           f"offset:{32 * kk}", "vmem_ld", {f"v{V_QOFF + rb}"}, regs("a", d, 4), vm=True))
    for rb in range(2):
        for kk in range(8):
            d = DO_A + 8 * kk + 4 * rb
            out.append(Ins(f"buffer_load_dwordx4 {areg(d, 4)}, {vreg(V_QOFF + rb)}, {s_in('dorsrc')}, 0 offen "
                           f"offset:{32 * kk}", "vmem_ld", {f"v{V_QOFF + rb}"}, regs("a", d, 4), vm=True))
    # K(0), V(0), K(1), V(1), V(2): the pre step waits for the Q / dO rows,
    # K(0) and V(0) only
    for kind, slot in (("k", 0), ("v", 0), ("k", 1), ("v", 1), ("v", 2)):
        for i in range(4):
            out += dma(kind, i, slot)
        out += desc_advance(kind)
    # dQ^T = 0 by eight MFMAs of zero operands
    z = V_MK
    out += [valu(f"v_mov_b32 {vreg(z + k)}, 0", set(), {f"v{z + k}"}) for k in range(4)]
    for blk in range(8):
        out.append(mfma(("a", DQ_A + 16 * blk), ("v", z), ("v", z), False))
    for kk in range(8):
        out.append(valu(f"v_xor_b32 {vreg(KOFF_V + kk)}, {32 * kk}, {vreg(D_V)}", {f"v{D_V}"},
                        {f"v{KOFF_V + kk}"}))
        out.append(valu(f"v_add_u32 {vreg(VOFF_V + kk)}, {V_RING}, {vreg(KOFF_V + kk)}", {f"v{KOFF_V + kk}"},
                        {f"v{VOFF_V + kk}"}))
    out.append(valu(f"v_mov_b32 {vreg(V_NINF)}, {NEG_INF_BITS:#x}", set(), {f"v{V_NINF}"}))
    # Q, dO, K(0) and V(0) have landed in every wave, and every wave has
    # read its inputs (V slot 3 is staged into by the pre step)
    out += [waitcnt(vm=12, lgkm=0), Ins("s_barrier", "barrier")]
    # The (-Delta, -Delta) pairs, row block 1's on the Q offsets, free now
    # that the Q / dO rows have landed.
    n0, n1 = V_NDLT
    out += [valu(f"v_xor_b32 {vreg(n1)}, 0x80000000, {vreg(V_DLT + 1)}", {f"v{V_DLT + 1}"}, {f"v{n1}"}),
            valu(f"v_xor_b32 {vreg(n1 + 1)}, 0x80000000, {vreg(V_DLT + 1)}", {f"v{V_DLT + 1}"}, {f"v{n1 + 1}"}),
            valu(f"v_xor_b32 {vreg(n0)}, 0x80000000, {vreg(V_DLT)}", {f"v{V_DLT}"}, {f"v{n0}"}),
            valu(f"v_mov_b32 {vreg(n0 + 1)}, {vreg(n0)}", {f"v{n0}"}, {f"v{n0 + 1}"})]
    return out


def epilogue():
    """dq rows: scale * dQ^T as bf16, staged per 32-row block through this
    wave's LDS region (rows at a 272-byte stride, then their byte offsets)
    so that each store writes 16 bytes of a whole 256-byte row; or, for a
    piece of a cut row tile, the fp32 partial as sixteen float4 units per
    lane and row block: unit 4 db + j at (16 rb + unit) KiB + 16 lane of the
    wave's part.  Returns the head (wait, branch to the piece stores), the
    whole-row stores and the piece stores."""
    u = "%="
    head = [waitcnt(vm=0, lgkm=0), salu(f"s_cmp_lg_u32 {s_in('piece')}, 0"),
            branch("s_cbranch_scc1", f"Lpart_{u}")]
    # every wave is past its last LDS read of the rings
    whole = [Ins("s_barrier", "barrier")]
    E, t5, t6, lane = 184, 189, 190, 191      # v[184:191]: addresses (the loop's dP^T tile is dead)
    whole += [
        valu(f"v_mbcnt_lo_u32_b32 {vreg(lane)}, -1, 0", set(), {f"v{lane}"}),
        valu(f"v_mbcnt_hi_u32_b32 {vreg(lane)}, -1, {vreg(lane)}", {f"v{lane}"}, {f"v{lane}"}),
        # E: write base (row lane & 31, 8 bytes per lane half); E+1: this
        # row's slot of the offset table; E+2: read base (row lane >> 4,
        # 16-byte chunk lane & 15); E+3: offset-table read base; E+4: 16 (lane & 15)
        valu(f"v_and_b32 {vreg(t5)}, 31, {vreg(lane)}", {f"v{lane}"}, {f"v{t5}"}),
        valu(f"v_lshrrev_b32 {vreg(t6)}, 5, {vreg(lane)}", {f"v{lane}"}, {f"v{t6}"}),
        valu(f"v_mul_u32_u24 {vreg(E)}, 0x110, {vreg(t5)}", {f"v{t5}"}, {f"v{E}"}),
        valu(f"v_lshl_add_u32 {vreg(E)}, {vreg(t6)}, 3, {vreg(E)}", {f"v{t6}", f"v{E}"}, {f"v{E}"}),
        valu(f"v_add_u32 {vreg(E)}, {s_in('ebase')}, {vreg(E)}", {f"v{E}"}, {f"v{E}"}),
        valu(f"v_lshl_add_u32 {vreg(E + 1)}, {vreg(t5)}, 2, {s_in('ebase')}", {f"v{t5}"}, {f"v{E + 1}"}),
        valu(f"v_add_u32 {vreg(E + 1)}, {32 * 272}, {vreg(E + 1)}", {f"v{E + 1}"}, {f"v{E + 1}"}),
        valu(f"v_lshrrev_b32 {vreg(t6)}, 4, {vreg(lane)}", {f"v{lane}"}, {f"v{t6}"}),
        valu(f"v_and_b32 {vreg(E + 4)}, 15, {vreg(lane)}", {f"v{lane}"}, {f"v{E + 4}"}),
        valu(f"v_lshlrev_b32 {vreg(E + 4)}, 4, {vreg(E + 4)}", {f"v{E + 4}"}, {f"v{E + 4}"}),
        valu(f"v_mul_u32_u24 {vreg(E + 2)}, 0x110, {vreg(t6)}", {f"v{t6}"}, {f"v{E + 2}"}),
        valu(f"v_add3_u32 {vreg(E + 2)}, {s_in('ebase')}, {vreg(E + 2)}, {vreg(E + 4)}",
             {f"v{E + 2}", f"v{E + 4}"}, {f"v{E + 2}"}),
        valu(f"v_lshl_add_u32 {vreg(E + 3)}, {vreg(t6)}, 2, {s_in('ebase')}", {f"v{t6}"}, {f"v{E + 3}"}),
        valu(f"v_add_u32 {vreg(E + 3)}, {32 * 272}, {vreg(E + 3)}", {f"v{E + 3}"}, {f"v{E + 3}"}),
    ]
    for rb in range(2):
        if rb == 1:
            whole.append(waitcnt(lgkm=0))     # row block 0's reads of the region are done
        for db in range(4):
            for j in range(4):
                a0 = DQ_A + 32 * db + 16 * rb + 4 * j
                tv = 8 * (4 * db + j) % 64   # rotate through v[0:63]
                for k in range(4):
                    whole.append(valu(f"v_accvgpr_read_b32 {vreg(tv + k)}, {areg(a0 + k)}", {f"a{a0 + k}"},
                                      {f"v{tv + k}"}))
                for k in range(4):
                    whole.append(valu(f"v_mul_f32 {vreg(tv + k)}, {s_in('scale')}, {vreg(tv + k)}",
                                      {f"v{tv + k}"}, {f"v{tv + k}"}))
                whole.append(valu(f"v_cvt_pk_bf16_f32 {vreg(tv + 4)}, {vreg(tv)}, {vreg(tv + 1)}",
                                  {f"v{tv}", f"v{tv + 1}"}, {f"v{tv + 4}"}))
                whole.append(valu(f"v_cvt_pk_bf16_f32 {vreg(tv + 5)}, {vreg(tv + 2)}, {vreg(tv + 3)}",
                                  {f"v{tv + 2}", f"v{tv + 3}"}, {f"v{tv + 5}"}))
                whole.append(Ins(f"ds_write_b64 {vreg(E)}, {vreg(tv + 4, 2)} offset:{64 * db + 16 * j}",
                                 "lds_w", {f"v{E}", f"v{tv + 4}", f"v{tv + 5}"}, set(), lgkm=True))
        # the row's byte offset (its lane-half term cleared; a row not
        # stored has an offset past the descriptor's range)
        whole.append(valu(f"v_and_b32 {vreg(t5)}, 0xfffffff7, {vreg(V_DQOFF + rb)}", {f"v{V_DQOFF + rb}"},
                          {f"v{t5}"}))
        whole.append(Ins(f"ds_write_b32 {vreg(E + 1)}, {vreg(t5)}", "lds_w", {f"v{E + 1}", f"v{t5}"}, set(),
                         lgkm=True))
        whole.append(waitcnt(lgkm=0))
        for i in range(8):
            whole.append(Ins(f"ds_read_b32 {vreg(64 + i)}, {vreg(E + 3)} offset:{16 * i}", "lds",
                             {f"v{E + 3}"}, {f"v{64 + i}"}, lgkm=True))
            whole.append(Ins(f"ds_read_b128 {vreg(72 + 4 * i, 4)}, {vreg(E + 2)} offset:{4 * 272 * i}", "lds",
                             {f"v{E + 2}"}, regs("v", 72 + 4 * i, 4), lgkm=True))
        for i in range(8):
            whole.append(valu(f"v_add_u32 {vreg(64 + i)}, {vreg(64 + i)}, {vreg(E + 4)}",
                              {f"v{64 + i}", f"v{E + 4}"}, {f"v{64 + i}"}))
            whole.append(Ins(f"buffer_store_dwordx4 {vreg(72 + 4 * i, 4)}, {vreg(64 + i)}, {s_in('dqrsrc')}, 0 "
                             f"offen", "vmem_st", regs("v", 72 + 4 * i, 4) | {f"v{64 + i}"}, set(), vm=True))
    whole.append(branch("s_branch", f"Lend_{u}", cond=False))
    t = V_TMP
    part = [valu(f"v_mbcnt_lo_u32_b32 {vreg(t)}, -1, 0", set(), {f"v{t}"}),
            valu(f"v_mbcnt_hi_u32_b32 {vreg(t)}, -1, {vreg(t)}", {f"v{t}"}, {f"v{t}"}),
            valu(f"v_lshlrev_b32 {vreg(t)}, 4, {vreg(t)}", {f"v{t}"}, {f"v{t}"})]
    for rb in range(2):
        for g in range(4):
            vo = 4 * rb + g      # v[0:7]: lane offsets of unit group g of row block rb
            part.append(valu(f"v_add_u32 {vreg(vo)}, {16384 * rb + 4096 * g}, {vreg(t)}", {f"v{t}"},
                             {f"v{vo}"}))
    for rb in range(2):
        for db in range(4):
            for j in range(4):
                unit = 4 * db + j
                a = DQ_A + 32 * db + 16 * rb + 4 * j
                vo = 4 * rb + unit // 4
                part.append(Ins(f"buffer_store_dwordx4 {areg(a, 4)}, {vreg(vo)}, {s_in('prsrc')}, 0 offen "
                                f"offset:{1024 * (unit % 4)}", "vmem_st", regs("a", a, 4) | {f"v{vo}"}, set(),
                                vm=True))
    return head, whole, part


def program():
    u = "%="
    blocks = [Block(f"Lpro_{u}", prologue() + [salu(f"s_cmp_le_i32 {sreg(S_N)}, 0"),
                                                  branch("s_cbranch_scc1", f"Lepi_{u}")])]
    blocks += step_blocks("p", 3, "pre", None)
    blocks.append(Block(f"Lr0_{u}", [salu(f"s_mov_b32 {sreg(S_R1)}, 1")]))
    for q in range(4):
        blocks.append(Block(f"Lt{q}_{u}", [salu(f"s_cmp_ge_i32 {sreg(S_R1)}, {sreg(S_N)}"),
                                          branch("s_cbranch_scc1", f"Llast{q}_{u}")]))
        blocks += step_blocks(f"f{q}", q, "full", f"Linc{q}_{u}")
        tail = [salu(f"s_add_u32 {sreg(S_R1)}, {sreg(S_R1)}, 1")]
        if q == 3:
            tail.append(branch("s_branch", f"Lt0_{u}", cond=False))
        blocks.append(Block(f"Linc{q}_{u}", tail))
    for q in range(4):
        bl = step_blocks(f"l{q}", q, "last", f"Lepi_{u}")
        bl[0].name = f"Llast{q}_{u}"
        blocks += bl
    head, whole, part = epilogue()
    blocks += [Block(f"Lepi_{u}", head), Block(f"Lwhole_{u}", whole), Block(f"Lpart_{u}", part),
               Block(f"Lend_{u}", [])]
    return blocks


def generate():
    blocks = program()
    waited = insert_waits(blocks)
    for b, w in zip(blocks, waited):
        b.ins = w
    padded = pad_program(blocks)
    lines = []
    for b, ins_list in zip(blocks, padded):
        lines.append(f"{b.name}:")
        for ins in ins_list:
            lines.append("  " + ins.text)
    return lines


def clobbers():
    c = [f"v{i}" for i in range(256)] + [f"a{i}" for i in range(256)]
    c += [f"s{i}" for i in range(S_FIRST, S_LASTC + 1)]
    c += ["vcc", "exec", "m0", "memory"]
    return c


def emit(path):
    lines = generate()
    with open(path, "w") as f:
        f.write("// Generated by gen_bwd_dq.py: the tile loop of bwd_dq_wide_kernel.  Do not edit.\n")
        f.write("#pragma once\n")
        f.write("#define SWATTN_BWD_DQ_ASM \\\n")
        for ln in lines:
            f.write(f'  "{ln}\\n" \\\n')
        f.write('  ""\n')
        f.write(f"#define SWATTN_BWD_DQ_LDS_BYTES {LDS_BYTES}\n")
        f.write(f"#define SWATTN_BWD_DQ_AUX_GROUPS {AUX_GROUPS}\n")
        f.write(f"#define SWATTN_BWD_DQ_EPI_REGION {EPI_REGION}\n")
        f.write("#define SWATTN_BWD_DQ_CLOBBERS \\\n  ")
        f.write(", ".join(f'"{x}"' for x in clobbers()))
        f.write("\n")
    return len(lines)


if __name__ == "__main__":
    n = emit(sys.argv[1])
    print(f"{n} lines")
