"""Generates the block loop of ``bwd_dkdv_wide_kernel`` as gfx950 assembly.

The arithmetic is the dK / dV part of the derivative of the reference branch
kernel (swiattn_gqa_prefill_varlen.py V:176-241; the reference itself is
forward-only, V:14-15): for each key j of a 256-key tile and each routed row
r whose range holds it, P = 2^(c q_r.k_j - LSE_r) with the forward's log2
LSE, dS = P (dO_r.v_j - Delta_r), both rounded to bf16 for the products,
dv_j = sum_r P dO_r and dk_j = scale * sum_r dS q_r.  Keys outside a row's
range get S = -inf, hence P = 0 and dS = 0.

Layout.  A workgroup owns a (256-key tile, KV head) pair: four waves of 64
keys (two 32-key halves "kh"), one wave per SIMD.  The dK^T and dV^T
accumulators (128 d x 64 keys each, fp32) fill the 256 AGPRs; the wave's K
rows (the B operands of S) sit in 64 VGPRs; the tile's V rows sit in LDS.
The 32-row blocks of rows that can see the tile (the full-branch blocks
from the last down, then the local ones from the first up) stream through
a four-slot LDS ring (Q block, dO block), gathered from the rows' positions
by 32-bit buffer offsets that bwd_prep_kernel writes into each block's
1 KiB info;
the info blocks (LSE, Delta, key bounds, row offsets) travel through a
four-slot ring, each wave loading its own copy, so that every info read is
a fixed register plus an immediate offset.  Four products per block,
in the forms whose accumulators are the next products' B operands:

  S    = Q K^T       (A: Q rows from LDS, B: K in VGPRs; lane = key)
  D    = Delta - dO V^T   (A: dO rows from LDS, B: -V rows from LDS, C: Delta)
  dV^T += dO^T P     (A: dO^T by transposing LDS reads, B: P packed)
  -dK^T += Q^T (P D) (A: Q^T by transposing LDS reads, B: P D = -dS packed)

Each wave negates its own V rows in LDS once (exact for bf16), and the dP
accumulation starts from each row's Delta (the MFMA's C operand), so D =
Delta - dP comes out of the matrix cores and -dS = P D costs one multiply;
the epilogue scales dK^T by -scale.

Step r (phase q = r mod 4) issues S(r+1), dP(r+1) (32 MFMAs), then
dV^T(r), dK^T(r) (32 MFMAs).  Its VALU work: the packing of dS(r) (before
dP(r+1) overwrites it), P = 2^(S c - LSE) and -dS = P D of block r+1 in
place (after the masking of block r+1 when some row of it does not
see every key of the wave), and the packing of P(r+1) (after dV^T(r) has
read P(r)).  It loads block r+4's info into info slot q and gathers block
r+3's rows into ring slot (q+3) % 4.

Register map (per lane; j = key in the half, hh = lane / 32):
  a[0:127]    dK^T accumulators, (db, kh) at 32 db + 16 kh
  a[128:255]  dV^T accumulators, likewise
  v[0:63]     K operands, (kh, kk) at 32 kh + 4 kk
  v[64:95]    S, kh at 64 + 16 kh (element e: row 8 (e >> 2) + 4 hh + (e & 3))
  v[96:127]   D = Delta - dP, likewise (-dS in place)
  v[128:143]  P operands (bf16), (kh, s2) at 128 + 8 kh + 4 s2
  v[144:159]  -dS operands, likewise
  v[160:183]  six operand staging sets
  v[184:255]  LDS addresses, LSE of four rows at a time, Delta of the
              block's rows (the C operand of D), mask temporaries, gather
              and store offsets
"""

from __future__ import annotations

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from gen_fwd_wide import (RSRC_WORD3, Block, Ins, areg, branch, insert_waits, mfma,  # noqa: E402
                          pad_program, regs, s_in, salu, schedule, sreg, valu, vreg, waitcnt)

# ---------------------------------------------------------------------------
# registers
# ---------------------------------------------------------------------------
DK_A, DV_A = 0, 128
KB_V = 0
S_V, D_V = 64, 96
PP_V, PD_V = 128, 144
ST_V, N_SETS = 160, 6
LEADM = 2                 # MFMAs between an operand's read and the first MFMA that takes it
AOFF_V = 184              # [kk] Q / dO row read address (ring slot 0, Q part)
VOFF_V = 192              # [kk] V row read address (key half 0)
TOFF_V = 200              # [db][a] transposing read address (ring slot 0, Q part, k-step 0)
V_LSE = 208               # [j' % 2][e]: LSE of row 8 j' + 4 hh + e
V_DC = 216                # [e]: Delta of row 8 (e >> 2) + 4 hh + (e & 3), the C operand of D
V_IRO = 232               # info ring + this lane's gather row offsets (slot 0)
V_ILH = 233               # info ring + 16 hh: this lane's rows (slot 0)
V_CH = 234                # [L] chunk offset of this lane's gather load L
V_GT = 236                # [L] gather offsets; the mask flag's read
V_KEY = 238               # this lane's key in half 0
V_MK = 240                # 240..247 mask temporaries
V_NINF = 248
V_L16 = 251               # 16 lane
V_TMP = 252
V_DKOFF = 253             # [kh] dK / dV row byte offset (+ 8 hh)
V_FA = 255                # the info ring (slot 0): the bounds summary reads

S_T0, S_T1, S_T2, S_T3 = 52, 53, 54, 55
S_R1 = 56                 # r + 1 for step r
S_N = 57                  # block count
S_MNEXT = 58              # block r + 1 needs the mask (set by step r - 1)
S_KW1 = 59                # the wave's last key + 1
S_PAIRS = (60, 62, 64, 66)
S_SOFF = 69
S_VRS = 72                # the V tile descriptor, advanced four rows per load
S_VB = 76                 # V bytes from the descriptor base to the tile's end
S_IS = 77                 # info slot of the info load
S_FIRST, S_LASTC = 52, 77

NEG_INF_BITS = 0xFF800000
SLOT_BYTES = 16384        # Q block + dO block
PART_DO = 8192
RING = 65536              # ring base relative to the V tile
INFO = RING + 4 * SLOT_BYTES
INFO_SLOTS = 4
LDS_BYTES = INFO + INFO_SLOTS * 1024
AUX_GROUPS = 6
AUX_OFF = RING + 2 * SLOT_BYTES   # ring slots 2-3 (the prologue gathers into 0-1)
IW_LSE, IW_DLT, IW_ST, IW_EN = 0, 32, 64, 96   # info word offsets
IW_MAXS, IW_MINE, IW_RO32 = 128, 129, 160

# ---------------------------------------------------------------------------
# operand loads and products
# ---------------------------------------------------------------------------


def st(o):
    return ST_V + 4 * (o % N_SETS)


def load_ins(ld, o, q):
    """LDS reads of operand load ld (index o in the step) for phase q: the
    step's S / dP block r+1 is in ring slot (q+1) % 4, its dV / dK block r
    in slot q."""
    kind = ld[0]
    dst = st(o)
    if kind in ("aq", "ad"):          # Q / dO rows of block r+1, k-step kk
        kk = ld[1]
        off = ((q + 1) % 4) * SLOT_BYTES + (PART_DO if kind == "ad" else 0)
        return [Ins(f"ds_read_b128 {vreg(dst, 4)}, {vreg(AOFF_V + kk)} offset:{off}", "lds",
                    {f"v{AOFF_V + kk}"}, regs("v", dst, 4), lgkm=True)]
    if kind == "bv":                  # V rows of key half kh, k-step kk
        kh, kk = ld[1], ld[2]
        return [Ins(f"ds_read_b128 {vreg(dst, 4)}, {vreg(VOFF_V + kk)} offset:{kh * 8192}", "lds",
                    {f"v{VOFF_V + kk}"}, regs("v", dst, 4), lgkm=True)]
    # "tq" / "td": Q^T / dO^T of block r, k-step s2 (16 rows), d block db
    s2, db = ld[1], ld[2]
    off = q * SLOT_BYTES + (PART_DO if kind == "td" else 0) + 4096 * s2
    out = []
    for half in range(2):
        adr = TOFF_V + 2 * db + half
        out.append(Ins(f"ds_read_b64_tr_b16 {vreg(dst + 2 * half, 2)}, {vreg(adr)} offset:{off}", "lds",
                       {f"v{adr}"}, regs("v", dst + 2 * half, 2), lgkm=True))
    return out


def step_ops(kind):
    """(loads, mfmas): loads in issue order; each MFMA names the loads it
    takes by index."""
    loads, mf = [], []
    if kind != "last":
        for kk in range(8):                         # S(r+1)
            loads.append(("aq", kk))
            a = len(loads) - 1
            for kh in range(2):
                mf.append(("s", kh, kk, a, None))
        for kk in range(8):                         # dP(r+1)
            loads.append(("ad", kk))
            a = len(loads) - 1
            for kh in range(2):
                loads.append(("bv", kh, kk))
                mf.append(("d", kh, kk, a, len(loads) - 1))
    if kind != "pre":
        for part in ("td", "tq"):                   # dV^T(r), then dK^T(r)
            for s2 in range(2):
                for db in range(4):
                    loads.append((part, s2, db))
                    a = len(loads) - 1
                    for kh in range(2):
                        mf.append((part, kh, (s2, db), a, None))
    return loads, mf


def mfma_ins(m):
    kind, kh, idx, a, b = m
    if kind == "s":
        kk = idx
        return mfma(("v", S_V + 16 * kh), ("v", st(a)), ("v", KB_V + 32 * kh + 4 * kk), kk > 0)
    if kind == "d":
        kk = idx
        if kk > 0:
            return mfma(("v", D_V + 16 * kh), ("v", st(a)), ("v", st(b)), True)
        # the chain starts from Delta (C operand in its own registers)
        dst, c = D_V + 16 * kh, V_DC
        ab = regs("v", st(a), 4) | regs("v", st(b), 4)
        return Ins(f"v_mfma_f32_32x32x16_bf16 {vreg(dst, 16)}, {vreg(st(a), 4)}, {vreg(st(b), 4)}, {vreg(c, 16)}",
                   "mfma", ab | regs("v", c, 16), regs("v", dst, 16),
                   mfma=(("v", dst), ab, regs("v", c, 16)))
    s2, db = idx
    if kind == "td":
        return mfma(("a", DV_A + 32 * db + 16 * kh), ("v", st(a)), ("v", PP_V + 8 * kh + 4 * s2), True)
    return mfma(("a", DK_A + 32 * db + 16 * kh), ("v", st(a)), ("v", PD_V + 8 * kh + 4 * s2), True)


# ---------------------------------------------------------------------------
# VALU work
# ---------------------------------------------------------------------------


def row_read(base, w0, jp, slot):
    """Four words (rows 8 j' + 4 hh .. +3) of the info field at word w0 of
    info slot `slot`, into base + 4 (j' % 2)."""
    d = base + 4 * (jp % 2)
    return Ins(f"ds_read_b128 {vreg(d, 4)}, {vreg(V_ILH)} offset:{1024 * slot + 4 * w0 + 32 * jp}", "lds",
               {f"v{V_ILH}"}, regs("v", d, 4), lgkm=True)


def exps(slot):
    """P = 2^(S c - LSE) in place, rows four at a time (their LSE read just
    before from info slot `slot`)."""
    out = []
    for jp in range(4):
        out.append(row_read(V_LSE, IW_LSE, jp, slot))
        for e in range(4 * jp, 4 * jp + 4):
            for kh in range(2):
                x = S_V + 16 * kh + e
                lse = V_LSE + 4 * (jp % 2) + (e & 3)
                out.append(valu(f"v_fma_f32 {vreg(x)}, {vreg(x)}, {s_in('c')}, -{vreg(lse)}",
                                {f"v{x}", f"v{lse}"}, {f"v{x}"}))
                out[-1].feeds_trans = True
                out.append(valu(f"v_exp_f32 {vreg(x)}, {vreg(x)}", {f"v{x}"}, {f"v{x}"}, trans=True))
    return out


def dss():
    """-dS = P D = P (Delta - dP) in place in the D registers."""
    out = []
    for e in range(16):
        for kh in range(2):
            x = S_V + 16 * kh + e
            d = D_V + 16 * kh + e
            out.append(valu(f"v_mul_f32 {vreg(d)}, {vreg(d)}, {vreg(x)}", {f"v{d}", f"v{x}"}, {f"v{d}"}))
    return out


def delta_reads(slot):
    """Delta of the block's rows into the C operand of D (element e = row
    8 (e >> 2) + 4 hh + (e & 3)), from info slot `slot`."""
    return [Ins(f"ds_read_b128 {vreg(V_DC + 4 * jp, 4)}, {vreg(V_ILH)} offset:{1024 * slot + 4 * IW_DLT + 32 * jp}",
                "lds", {f"v{V_ILH}"}, regs("v", V_DC + 4 * jp, 4), lgkm=True) for jp in range(4)]


def packs(src, dst):
    """bf16 operands (kh, s2): register m of (kh, s2) holds elements 8 s2 +
    2 m, +1 of half kh."""
    out = []
    for kh in range(2):
        for s2 in range(2):
            for m in range(4):
                a = src + 16 * kh + 8 * s2 + 2 * m
                d = dst + 8 * kh + 4 * s2 + m
                out.append(valu(f"v_cvt_pk_bf16_f32 {vreg(d)}, {vreg(a)}, {vreg(a + 1)}",
                                {f"v{a}", f"v{a + 1}"}, {f"v{d}"}))
    return out


def mask(slot):
    """S of block r+1 outside each row's [start, end) set to -inf: for each
    group j' of four rows, key - start < end - start (unsigned) keeps it;
    the key of half 1 is the key of half 0 plus 32."""
    out = []
    for jp in range(4):
        out += _mask_group(jp, slot)
    return out


def _mask_group(jp, slot):
    # starts into MK[0:4] (j' even) or MK[4:8] (j' odd); ends into the
    # other four, each group's registers free again once its compares ran
    st_r = V_MK + 4 * (jp % 2)
    en_r = V_MK + 4 * (1 - jp % 2)
    base = 1024 * slot
    out = [Ins(f"ds_read_b128 {vreg(st_r, 4)}, {vreg(V_ILH)} offset:{base + 4 * IW_ST + 32 * jp}", "lds",
               {f"v{V_ILH}"}, regs("v", st_r, 4), lgkm=True),
           Ins(f"ds_read_b128 {vreg(en_r, 4)}, {vreg(V_ILH)} offset:{base + 4 * IW_EN + 32 * jp}", "lds",
               {f"v{V_ILH}"}, regs("v", en_r, 4), lgkm=True)]
    for e in range(4):
        sr, er = st_r + e, en_r + e
        out += [valu(f"v_sub_u32 {vreg(er)}, {vreg(er)}, {vreg(sr)}", {f"v{er}", f"v{sr}"}, {f"v{er}"}),
                valu(f"v_sub_u32 {vreg(sr)}, {vreg(V_KEY)}, {vreg(sr)}", {f"v{V_KEY}", f"v{sr}"}, {f"v{sr}"})]
        for kh in range(2):
            p = S_PAIRS[kh]
            x = S_V + 16 * kh + 4 * jp + e
            if kh == 1:
                out.append(valu(f"v_add_u32 {vreg(sr)}, 32, {vreg(sr)}", {f"v{sr}"}, {f"v{sr}"}))
            out += [valu(f"v_cmp_gt_u32_e64 {sreg(p, 2)}, {vreg(er)}, {vreg(sr)}", {f"v{er}", f"v{sr}"},
                         {f"s{p}", f"s{p + 1}"}),
                    valu(f"v_cndmask_b32_e64 {vreg(x)}, {vreg(V_NINF)}, {vreg(x)}, {sreg(p, 2)}",
                         {f"v{x}", f"v{V_NINF}"}, {f"v{x}"}, mask_rd={f"s{p}", f"s{p + 1}"})]
    return out


# ---------------------------------------------------------------------------
# block bookkeeping: packed block of list index a, info loads, row gathers,
# the mask flag
# ---------------------------------------------------------------------------


def block_index(sdst, rel):
    """sdst = packed block of list index a = min(r + rel, n - 1) (S_R1 = r
    + 1).  The full-branch blocks come first, from the last down (pbf =
    the last one's packed index), so that the pairs an XCD runs at once,
    which share their full rows' later blocks, read the same block at about
    the same time; then the local blocks from the first up: a + pb1 (pb1
    already less n0; pb1n = pb1 + n0)."""
    return [salu(f"s_add_u32 {sreg(sdst)}, {sreg(S_R1)}, {rel - 1}"),
            salu(f"s_add_u32 {sreg(S_T3)}, {sreg(S_N)}, -1"),
            salu(f"s_min_i32 {sreg(sdst)}, {sreg(sdst)}, {sreg(S_T3)}"),
            salu(f"s_sub_u32 {sreg(S_T3)}, {s_in('pbf')}, {sreg(sdst)}"),
            salu(f"s_add_u32 {sreg(sdst)}, {sreg(sdst)}, {s_in('pb1')}"),
            salu(f"s_cmp_lt_i32 {sreg(sdst)}, {s_in('pb1n')}"),
            salu(f"s_cselect_b32 {sreg(sdst)}, {sreg(S_T3)}, {sreg(sdst)}")]


def info_dma(rel, slot):
    """Block r+rel's 1 KiB info into info slot `slot` (every wave its own
    copy, so that each wave waits only for its own load).  The whole offset
    is in the lane's offset register, where the descriptor's range check
    sees it."""
    out = block_index(S_T0, rel)
    out += [salu(f"s_lshl_b32 {sreg(S_T0)}, {sreg(S_T0)}, 10"),
            valu(f"v_add_u32 {vreg(V_TMP)}, {sreg(S_T0)}, {vreg(V_L16)}", {f"s{S_T0}", f"v{V_L16}"},
                 {f"v{V_TMP}"}),
            salu(f"s_add_u32 m0, {s_in('info0')}, {1024 * slot}", wr={"m0"}),
            Ins(f"buffer_load_dwordx4 {vreg(V_TMP)}, {s_in('irsrc')}, 0 offen lds", "dma",
                {"m0", f"v{V_TMP}"}, set(), vm=True)]
    return out


def gather(slot, islot):
    """This wave's share of a block's rows into ring slot `slot`, from the
    row offsets in info slot `islot`: loads L = 2 w, 2 w + 1 of the Q part
    and of the dO part (rows 4 L .. 4 L + 3), each lane fetching its chunk
    at its row's offset."""
    out = []
    for L in range(2):
        out.append(Ins(f"ds_read_b32 {vreg(V_GT + L)}, {vreg(V_IRO)} offset:{1024 * islot + 16 * L}", "lds",
                       {f"v{V_IRO}"}, {f"v{V_GT + L}"}, lgkm=True))
    for L in range(2):
        out.append(valu(f"v_add_u32 {vreg(V_GT + L)}, {vreg(V_GT + L)}, {vreg(V_CH + L)}",
                        {f"v{V_GT + L}", f"v{V_CH + L}"}, {f"v{V_GT + L}"}))
    for part, rs in ((0, "qrsrc"), (PART_DO, "dorsrc")):
        for L in range(2):
            base = RING + slot * SLOT_BYTES + part
            out += [salu(f"s_add_u32 m0, {s_in('wl')}, {base + 1024 * L}", wr={"m0"}),
                    Ins(f"buffer_load_dwordx4 {vreg(V_GT + L)}, {s_in(rs)}, 0 offen lds", "dma",
                        {f"v{V_GT + L}", "m0"}, set(), vm=True)]
    return out


def mask_flag(islot):
    """S_MNEXT = the block in info slot `islot` has a row whose range does
    not hold every key of the wave (from its bounds summary)."""
    return [Ins(f"ds_read_b64 {vreg(V_GT, 2)}, {vreg(V_FA)} offset:{1024 * islot + 4 * IW_MAXS}", "lds",
                {f"v{V_FA}"}, regs("v", V_GT, 2), lgkm=True),
            valu(f"v_readfirstlane_b32 {sreg(S_T2)}, {vreg(V_GT)}", {f"v{V_GT}"}, {f"s{S_T2}"}),
            valu(f"v_readfirstlane_b32 {sreg(S_T3)}, {vreg(V_GT + 1)}", {f"v{V_GT + 1}"}, {f"s{S_T3}"}),
            Ins("s_nop 4", "nop"),
            salu(f"s_cmp_gt_i32 {sreg(S_T2)}, {s_in('kw0')}", {f"s{S_T2}"}),
            salu(f"s_cselect_b32 {sreg(S_MNEXT)}, 1, 0", wr={f"s{S_MNEXT}"}),
            salu(f"s_cmp_lt_i32 {sreg(S_T3)}, {sreg(S_KW1)}", {f"s{S_T3}", f"s{S_KW1}"}),
            salu(f"s_cselect_b32 {sreg(S_T2)}, 1, 0", wr={f"s{S_T2}"}),
            salu(f"s_or_b32 {sreg(S_MNEXT)}, {sreg(S_MNEXT)}, {sreg(S_T2)}", {f"s{S_MNEXT}", f"s{S_T2}"},
                 {f"s{S_MNEXT}"})]


# ---------------------------------------------------------------------------
# steps
# ---------------------------------------------------------------------------
# Step r (phase q): S(r+1), dP(r+1) from block r+1's rows in ring slot
# (q+1) % 4, dV^T(r), dK^T(r) from block r's rows in slot q.  Block b's info
# is in info slot b % 4.  The step first loads block r+4's info into info
# slot q (block r's, last read by step r-1), then gathers block r+3 into
# ring slot (q+3) % 4 (block r-1's, last read by step r-1) and reads block
# r+2's bounds summary for the next step's mask choice.


def _spread(items, nm, lo=0.1, hi=0.75):
    """Side positions for a list of instruction groups, spread over the
    MFMA slots between fractions lo and hi of the step."""
    n = len(items)
    out = {}
    for k, it in enumerate(items):
        pos = int(nm * (lo + (hi - lo) * k / max(1, n - 1)))
        out.setdefault(max(1, min(nm - 1, pos)), []).extend(it)
    return out


def step_code(q, kind, masked):
    loads, mfs = step_ops(kind)
    mf = [mfma_ins(m) for m in mfs]
    nm = len(mf)
    first_use, last_use = {}, {}
    for i, m in enumerate(mfs):
        for a in (m[3], m[4]):
            if a is not None:
                first_use.setdefault(a, i)
                last_use[a] = i
    # operand o is read LEADM MFMAs before its first use, but only once the
    # previous load of its staging set has been taken by its last MFMA
    reads = {}
    for o, ld in enumerate(loads):
        at = first_use[o] - LEADM
        if o >= N_SETS:
            at = max(at, last_use[o - N_SETS] + 1)
        at = max(at, 0)
        reads.setdefault(at, []).extend(load_ins(ld, o, q))
    side_extra = {}
    if kind != "last":
        # the info load is this step's first memory operation (the next
        # step's barrier waits for it and lets the four gathers run on)
        g = gather((q + 3) % 4, (q + 3) % 4)
        groups = [info_dma(4, q), mask_flag((q + 2) % 4), g[:4]] + [g[4 + 2 * k: 6 + 2 * k] for k in range(4)]
        side_extra = _spread(groups, nm, 0.02, 0.6)

    def side(i):
        return side_extra.get(i, []) + reads.get(i, [])

    carried = []
    if kind != "pre":
        carried = packs(D_V, PD_V)           # -dS(r), before D(r+1) overwrites it
    if kind != "last":
        carried += delta_reads((q + 1) % 4)  # block r+1's Delta, before D(r+1) starts from it
    vl = list(carried)
    if kind != "last":
        islot = (q + 1) % 4
        if masked:
            vl += mask(islot)
        vl += exps(islot) + dss() + packs(S_V, PP_V)
    o, _ = schedule(mf, vl, side, carry=False, n_carried=len(carried), lead_cap=4, one_feed=True)
    return o


def step_blocks(tag, q, kind, end_label):
    u = "%="
    if kind == "pre":
        return [Block(f"L{tag}_a_{u}", step_code(q, "pre", True))]
    # block r+1's rows (gathered two steps ago) have landed in every wave,
    # and so has the info of block r+3 (the previous step's first load);
    # the previous step's four gathers may still be in flight
    blocks = [Block(f"L{tag}_s_{u}", [waitcnt(vm=4, lgkm=0), Ins("s_barrier", "barrier")])]
    if kind == "last":
        blocks.append(Block(f"L{tag}_a_{u}", step_code(q, "last", False)
                            + [branch("s_branch", end_label, cond=False)]))
        return blocks
    blocks.append(Block(f"L{tag}_mt_{u}", [salu(f"s_cmp_lg_u32 {sreg(S_MNEXT)}, 0"),
                                           branch("s_cbranch_scc1", f"L{tag}_am_{u}")]))
    blocks.append(Block(f"L{tag}_au_{u}", step_code(q, "full", False)
                        + [branch("s_branch", end_label, cond=False)]))
    blocks.append(Block(f"L{tag}_am_{u}", step_code(q, "full", True)))
    return blocks


def prologue():
    """Per-lane inputs from LDS, K rows into their VGPRs, the V tile into
    LDS, dK^T = dV^T = 0, the info of blocks 0..3; once blocks 0-1's info
    has landed their rows, block 0's info read base and block 1's mask
    flag; wait and barrier."""
    out = [salu("s_mov_b64 exec, -1"), Ins("s_nop 7", "nop")]
    t = V_TMP
    out += [valu(f"v_mbcnt_lo_u32_b32 {vreg(t)}, -1, 0", set(), {f"v{t}"}),
            valu(f"v_mbcnt_hi_u32_b32 {vreg(t)}, -1, {vreg(t)}", {f"v{t}"}, {f"v{t}"}),
            valu(f"v_lshlrev_b32 {vreg(V_L16)}, 4, {vreg(t)}", {f"v{t}"}, {f"v{V_L16}"}),
            valu(f"v_add_u32 {vreg(t)}, {s_in('aux')}, {vreg(V_L16)}", {f"v{V_L16}"}, {f"v{t}"})]
    # input groups (four words per lane): 0 K load offsets (kh), dK / dV row
    # offsets (kh); 1 A and V read address bases, gather chunk offsets (L);
    # 2-3 transposing read addresses; 4 V tile DMA offsets (i mod 4); 5 the
    # key of half 0, 16 hh, this lane's gather row-offset position, unused
    dst = {0: S_V, 1: S_V + 4, 2: TOFF_V, 3: TOFF_V + 4, 4: S_V + 8, 5: S_V + 12}
    for g in range(AUX_GROUPS):
        d = dst[g]
        out.append(Ins(f"ds_read_b128 {vreg(d, 4)}, {vreg(t)} offset:{g * 1024}", "lds", {f"v{t}"},
                       regs("v", d, 4), lgkm=True))
    out += [salu(f"s_mov_b32 {sreg(S_N)}, {s_in('nblk')}"),
            salu(f"s_add_u32 {sreg(S_KW1)}, {s_in('kw0')}, 64"),
            salu(f"s_mov_b32 {sreg(S_R1)}, 0"),
            salu(f"s_mov_b64 {sreg(S_VRS, 2)}, {s_in('vbase')}"),
            salu(f"s_mov_b32 {sreg(S_VB)}, {s_in('vbytes')}"),
            salu(f"s_max_i32 {sreg(S_VRS + 2)}, {sreg(S_VB)}, 0"),
            salu(f"s_mov_b32 {sreg(S_VRS + 3)}, {RSRC_WORD3:#x}")]
    # K rows: (kh, kk) at 32 kh + 4 kk
    for kh in range(2):
        for kk in range(8):
            d = KB_V + 32 * kh + 4 * kk
            out.append(Ins(f"buffer_load_dwordx4 {vreg(d, 4)}, {vreg(S_V + kh)}, {s_in('krsrc')}, 0 offen "
                           f"offset:{32 * kk}", "vmem_ld", {f"v{S_V + kh}"}, regs("v", d, 4), vm=True))
    # the V tile: this wave's 64 rows, four per load, the descriptor moved
    # on four rows per load (the rows past the keys' end fall outside it)
    for i in range(16):
        if i:
            out += [salu(f"s_add_u32 {sreg(S_VRS)}, {sreg(S_VRS)}, {s_in('krow4')}"),
                    salu(f"s_addc_u32 {sreg(S_VRS + 1)}, {sreg(S_VRS + 1)}, 0"),
                    salu(f"s_sub_i32 {sreg(S_VB)}, {sreg(S_VB)}, {s_in('krow4')}"),
                    salu(f"s_max_i32 {sreg(S_VRS + 2)}, {sreg(S_VB)}, 0")]
        out += [salu(f"s_add_u32 m0, {s_in('vl')}, {1024 * i}", wr={"m0"}),
                Ins(f"buffer_load_dwordx4 {vreg(S_V + 8 + (i % 4))}, {sreg(S_VRS, 4)}, 0 offen lds",
                    "dma", {f"v{S_V + 8 + (i % 4)}", "m0"} | regs("s", S_VRS, 4), set(), vm=True)]
    # per-lane state from the inputs
    out += [valu(f"v_mov_b32 {vreg(V_DKOFF + kh)}, {vreg(S_V + 2 + kh)}", {f"v{S_V + 2 + kh}"},
                 {f"v{V_DKOFF + kh}"}) for kh in range(2)]
    out += [valu(f"v_mov_b32 {vreg(V_CH + L)}, {vreg(S_V + 6 + L)}", {f"v{S_V + 6 + L}"}, {f"v{V_CH + L}"})
            for L in range(2)]
    out += [valu(f"v_mov_b32 {vreg(V_KEY)}, {vreg(S_V + 12)}", {f"v{S_V + 12}"}, {f"v{V_KEY}"}),
            valu(f"v_add_u32 {vreg(V_ILH)}, {s_in('info0')}, {vreg(S_V + 13)}", {f"v{S_V + 13}"},
                 {f"v{V_ILH}"}),
            valu(f"v_add_u32 {vreg(V_IRO)}, {s_in('info0')}, {vreg(S_V + 14)}", {f"v{S_V + 14}"},
                 {f"v{V_IRO}"}),
            valu(f"v_mov_b32 {vreg(V_FA)}, {s_in('info0')}", set(), {f"v{V_FA}"})]
    for kk in range(8):
        out.append(valu(f"v_xor_b32 {vreg(AOFF_V + kk)}, {32 * kk}, {vreg(S_V + 4)}", {f"v{S_V + 4}"},
                        {f"v{AOFF_V + kk}"}))
        out.append(valu(f"v_xor_b32 {vreg(VOFF_V + kk)}, {32 * kk}, {vreg(S_V + 5)}", {f"v{S_V + 5}"},
                        {f"v{VOFF_V + kk}"}))
    out.append(valu(f"v_mov_b32 {vreg(V_NINF)}, {NEG_INF_BITS:#x}", set(), {f"v{V_NINF}"}))
    # dK^T = dV^T = 0 by sixteen MFMAs of zero operands
    z = V_MK
    out += [valu(f"v_mov_b32 {vreg(z + k)}, 0", set(), {f"v{z + k}"}) for k in range(4)]
    for blk in range(16):
        out.append(mfma(("a", 16 * blk), ("v", z), ("v", z), False))
    # info of blocks 0..2 into info slots 0..2 (S_R1 = 0 here: list index
    # r + rel with r = -1)
    for b in range(3):
        out += info_dma(b + 1, b)
    # blocks 0-1's info has landed (this wave's own loads; 2 may still be in
    # flight), and every wave has read its inputs
    out += [waitcnt(vm=1, lgkm=0), Ins("s_barrier", "barrier")]
    # -V: this wave's 64 V rows (the only ones it reads) negated in place,
    # 16 bytes per lane and read
    t2 = S_V + 16
    out.append(valu(f"v_add_u32 {vreg(V_TMP)}, {s_in('vl')}, {vreg(V_L16)}", {f"v{V_L16}"}, {f"v{V_TMP}"}))
    for i in range(16):
        d = t2 + 4 * (i % 8)
        out.append(Ins(f"ds_read_b128 {vreg(d, 4)}, {vreg(V_TMP)} offset:{1024 * i}", "lds", {f"v{V_TMP}"},
                       regs("v", d, 4), lgkm=True))
        for k in range(4):
            out.append(valu(f"v_xor_b32 {vreg(d + k)}, 0x80008000, {vreg(d + k)}", {f"v{d + k}"}, {f"v{d + k}"}))
        out.append(Ins(f"ds_write_b128 {vreg(V_TMP)}, {vreg(d, 4)} offset:{1024 * i}", "lds_w",
                       {f"v{V_TMP}"} | regs("v", d, 4), set(), lgkm=True))
    out += gather(0, 0) + gather(1, 1)
    out += mask_flag(1)
    # block 0's rows have landed in every wave, and block 2's info (block
    # 1's four gathers may still be in flight)
    out += [waitcnt(vm=4), Ins("s_barrier", "barrier")]
    return out


def epilogue():
    """dK = scale dK^T and dV = dV^T as bf16 rows, four values per store, at
    each lane's key row (keys past the end fall outside the descriptors); or,
    for one split of a pair's row blocks, the fp32 partials for
    bwd_dkdv_reduce_kernel: key half kh of the wave is the reduce's wave
    2 w + kh, dK^T block db elements 4 j .. 4 j + 3 its unit 4 db + j (with
    the sign of dS^T Q: the loop accumulated its negative) and dV^T's unit
    16 + 4 db + j, at (32 kh + unit) KiB + 16 lane of the wave's part.
    Returns the head (wait, branch to the partial stores), the row stores
    and the partial stores."""
    u = "%="
    head = [waitcnt(vm=0, lgkm=0), salu(f"s_cmp_lg_u32 {s_in('split')}, 0"),
            branch("s_cbranch_scc1", f"Lpart_{u}")]
    part = [valu(f"v_mbcnt_lo_u32_b32 {vreg(V_TMP)}, -1, 0", set(), {f"v{V_TMP}"}),
            valu(f"v_mbcnt_hi_u32_b32 {vreg(V_TMP)}, -1, {vreg(V_TMP)}", {f"v{V_TMP}"}, {f"v{V_TMP}"}),
            valu(f"v_lshlrev_b32 {vreg(V_TMP)}, 4, {vreg(V_TMP)}", {f"v{V_TMP}"}, {f"v{V_TMP}"})]
    for kh in range(2):
        for g in range(8):
            vo = 8 * kh + g      # v[0:15]: lane offsets of unit group g of key half kh
            part.append(valu(f"v_add_u32 {vreg(vo)}, {32768 * kh + 4096 * g}, {vreg(V_TMP)}", {f"v{V_TMP}"},
                             {f"v{vo}"}))
    for kh in range(2):
        for db in range(4):
            for j in range(4):
                unit = 4 * db + j
                a = DK_A + 32 * db + 16 * kh + 4 * j
                t = 16 + 4 * ((4 * db + j) % 8)
                for k in range(4):
                    part.append(valu(f"v_accvgpr_read_b32 {vreg(t + k)}, {areg(a + k)}", {f"a{a + k}"},
                                     {f"v{t + k}"}))
                for k in range(4):
                    part.append(valu(f"v_xor_b32 {vreg(t + k)}, 0x80000000, {vreg(t + k)}", {f"v{t + k}"},
                                     {f"v{t + k}"}))
                vo = 8 * kh + unit // 4
                part.append(Ins(f"buffer_store_dwordx4 {vreg(t, 4)}, {vreg(vo)}, {s_in('prsrc')}, 0 offen "
                                f"offset:{1024 * (unit % 4)}", "vmem_st", regs("v", t, 4) | {f"v{vo}"}, set(),
                                vm=True))
                unit = 16 + 4 * db + j
                a = DV_A + 32 * db + 16 * kh + 4 * j
                vo = 8 * kh + unit // 4
                part.append(Ins(f"buffer_store_dwordx4 {areg(a, 4)}, {vreg(vo)}, {s_in('prsrc')}, 0 offen "
                                f"offset:{1024 * (unit % 4)}", "vmem_st", regs("a", a, 4) | {f"v{vo}"}, set(),
                                vm=True))
    out = []
    for acc, rs, scl in ((DK_A, "dkrsrc", True), (DV_A, "dvrsrc", False)):
        for kh in range(2):
            for db in range(4):
                tv = 64 + 16 * ((2 * kh + db) % 4)
                for k in range(16):
                    a = acc + 32 * db + 16 * kh + k
                    out.append(valu(f"v_accvgpr_read_b32 {vreg(tv + k)}, {areg(a)}", {f"a{a}"}, {f"v{tv + k}"}))
                if scl:
                    # the loop accumulated -dK^T
                    for k in range(16):
                        out.append(valu(f"v_mul_f32 {vreg(tv + k)}, -{s_in('scale')}, {vreg(tv + k)}",
                                        {f"v{tv + k}"}, {f"v{tv + k}"}))
                for jj in range(4):
                    for k in range(2):
                        out.append(valu(f"v_cvt_pk_bf16_f32 {vreg(tv + 4 * jj + k)}, {vreg(tv + 4 * jj + 2 * k)}, "
                                        f"{vreg(tv + 4 * jj + 2 * k + 1)}",
                                        {f"v{tv + 4 * jj + 2 * k}", f"v{tv + 4 * jj + 2 * k + 1}"},
                                        {f"v{tv + 4 * jj + k}"}))
                    out.append(Ins(f"buffer_store_dwordx2 {vreg(tv + 4 * jj, 2)}, {vreg(V_DKOFF + kh)}, "
                                   f"{s_in(rs)}, 0 offen offset:{64 * db + 16 * jj}", "vmem_st",
                                   regs("v", tv + 4 * jj, 2) | {f"v{V_DKOFF + kh}"}, set(), vm=True))
    out.append(branch("s_branch", f"Lend_{u}", cond=False))
    return head, out, part


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
        f.write("// Generated by gen_bwd_dkdv.py: the block loop of bwd_dkdv_wide_kernel.  Do not edit.\n")
        f.write("#pragma once\n")
        f.write("#define SWATTN_BWD_DKDV_ASM \\\n")
        for ln in lines:
            f.write(f'  "{ln}\\n" \\\n')
        f.write('  ""\n')
        f.write(f"#define SWATTN_BWD_DKDV_LDS_BYTES {LDS_BYTES}\n")
        f.write(f"#define SWATTN_BWD_DKDV_AUX_GROUPS {AUX_GROUPS}\n")
        f.write(f"#define SWATTN_BWD_DKDV_AUX_OFF {AUX_OFF}\n")
        f.write(f"#define SWATTN_BWD_DKDV_INFO_OFF {INFO}\n")
        f.write(f"#define SWATTN_BWD_DKDV_RING_OFF {RING}\n")
        f.write("#define SWATTN_BWD_DKDV_CLOBBERS \\\n  ")
        f.write(", ".join(f'"{x}"' for x in clobbers()))
        f.write("\n")
    return len(lines)


if __name__ == "__main__":
    n = emit(sys.argv[1])
    print(f"{n} lines")
