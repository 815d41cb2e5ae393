"""Generates the tile loop of ``fwd_wide_kernel`` as gfx950 assembly.

Reference tags: V = swiattn_gqa_prefill_varlen.py.  The arithmetic is the
reference branch kernel's hot loop (V:176-241): S = Q K^T, an online softmax
in base 2 with c = sm_scale * log2(e) (V:207-221), P rounded to bf16 for P V
while the row sum keeps the fp32 P (V:219-225), O = acc / l and
LSE = log2(l) + m * c (V:236-241), written back to the listed rows only
(V:243-249).

Why generated assembly.  A work item here is 256 rows, 64 per wave, one
wave per SIMD.  Per lane that needs the O accumulator (128 fp32), the Q^T
operands (64 registers), two S tiles for the software pipeline (128), the
packed P tile (32) and the K / V^T operand staging: more than the 256
VGPRs a compiler-allocated kernel gets, and the compiler's MFMA register
form is chosen per function, so it cannot keep O in AGPRs while S lives in
VGPRs.  Written out here, O, Q^T and the LDS operands live in AGPRs (the
matrix cores read and accumulate there directly) and S / P in VGPRs.

Issue budget.  One wave per SIMD issues everything in order, and measured
on gfx950 a wave issues about one instruction per five to six cycles, so
an MFMA slot (32 cycles for a 32x32x16 bf16 MFMA) holds about five other
instructions before the matrix core waits.  A step (one 64-key tile: 64
MFMAs) has about 230 VALU instructions of softmax that cannot be avoided
(two per exponential, the bf16 packing, the fp32 row sums, the checks;
about 280 where the running max is taken), so everything else is kept off
the path: the K and V^T rings have
four slots each and the loop is unrolled four steps, so every LDS operand
address is a base register plus an immediate offset; the buffer
descriptors of the global -> LDS copies advance with four scalar
instructions each; the two lanes of a row share one running-max update;
LDS waits cover two operand reads where the second is old enough.  Rules
from single-wave microbenchmarks: an exponential placed first behind an
MFMA can stall the next one, so each MFMA slot takes at most one
exponential and never as its first VALU instruction; a 64-key tile has 64
exponentials and 64 MFMAs, so the exponentials spread over both GEMMs.

Schedule.  The online softmax runs on 32-key halves of each tile (h = 0,
1; the running max moves at most per half).  The running max is kept as
n = -m c; a half's max x moves it only when d = x c + n exceeds 8 (P then
stays below 2^8 without a move), and the rescale exponent e is d or 0.
Each lane keeps the partial row sum of its own 16 keys of each half; the
two lanes of a row are added once, at the end.

The pre step (tile 0) and step 0 (tile 1) take that running max exactly,
so every row whose range starts within an item's first two tiles has a
finite max.  The steps after them take none: they exponentiate with n as
it stands and check each half afterwards.  Every lane's sum of its 16 P of
each row block must be at most 8192 (so every P is, as the online softmax
needs); a half that fails (the scores jumped, a row met its first key
late, or 2^x left the fp32 range) branches to an out-of-line routine that
fetches the tile's K rows from memory, recomputes the half's scores with
the same MFMAs in the same order, masks them, takes the exact running max
(whose O, l rescale then follows at the step's rescale point) and redoes
the exponentials, packing and sums.  A row whose max moved there from a
finite value had later exponentials taken with the old max: half 0's
recomputation forces half 1's check to fail (and the next tile's half 0),
half 1's the next tile's.

A step (tile j) starts with P(j) half 0 exponentiated, packed and its
sums' first level formed, and the first 16 exponentials of P(j) half 1
taken.  It is then:

  A  (32 MFMAs, S(j+1) half 0 then half 1):  the last 16 exponentials of
     P(j) half 1, the rest of half 0's lane sums and its check; once S(j+1)
     half 0 is final, its first 16 exponentials; then packing and lane sums
     of P(j) half 1 (what is left of them carries on);
  -- recompute P(j) half 0 when its check failed, O, l *= 2^-e(j, 0) when
     some row's max moved in half 0 of tile j (rare, out of line) --
  B1 (16 MFMAs, P(j) V(j) half 0):  half 0's sums added to l, the last 16
     exponentials of S(j+1) half 0, the rest of half 1 and its check;
  -- the same for half 1 of tile j --
  B2 (16 MFMAs, P(j) V(j) half 1):  half 1's sums added to l, the first 16
     exponentials of S(j+1) half 1, packing and first sum level of S(j+1)
     half 0; then the next step's first K and V^T operands are read
     (before its barrier).

Each half's packing and sums thus get about 32 MFMA slots before its
check.  The first exponentials of S(j+1) half 0 are taken before P(j)
half 0's check, so a recomputation of half 0 that moves a row's max from
a finite value forces the next tile's half-0 check too.  Step 0 takes the
running max of S(j+1) half 0 in A (before its exponentials) and of half 1
in B1, has no checks, and applies O, l *= 2^-e at the step's start and
between B1 and B2.  Work a block cannot fit moves on to the next one, but
never past a check the work precedes or a rescale it must precede, nor
past a step's end.

The output is one inline-asm string for ``swattn_fwd.hip``.  The generator
places each block's VALU work into its MFMA slots with a list scheduler,
inserts the ``s_waitcnt`` counts for its LDS and memory loads, and pads
with ``s_nop`` wherever gfx950 needs independent instructions between
dependent ones (the rules at the end, checked over the control-flow graph
so that every path is covered).

Register map (per lane; "rb" = row block 0/1 of the wave's 64 rows, "h" =
32-key half of a 64-key tile, "db" = 32-wide block of head_dim; "combined"
values hold row block 0 in lanes 0-31 and row block 1 in lanes 32-63):
  a[0:127]    O^T accumulators, block (db, rb) at a[32 db + 16 rb]
  a[128:191]  Q^T operands, k-step kk (16 of head_dim), rb at a[128 + 8 kk + 4 rb]
  a[192:223]  K operands, eight sets (one per (h, kk) read)
  a[224:247]  V^T operands, six sets
  v[0:63], v[64:127]   S tiles (ping-pong), (rb, h) at +32 rb + 16 h
  v[128:159]  P^T operands (bf16), k-step s2 (16 keys), rb at v[128 + 8 s2 + 4 rb]
  v[160:167]  K operand LDS addresses (slot 0) per kk; v[168:171] V^T per s2
  v[172:215]  row state and temporaries
  v[216:255]  left to the compiler (the asm's inputs)
"""

from __future__ import annotations

import re
import sys

# ---------------------------------------------------------------------------
# registers
# ---------------------------------------------------------------------------
O_A, Q_A, KOP_A, VOP_A = 0, 128, 192, 224
K_SETS, V_SETS = 8, 6      # LDS operand sets in flight
S_V = (0, 64)
PK_V = 128
KOFF_V, VOFF_V = 160, 168
V_L = 172                            # [rb] this lane's partial row sum
V_AL = 174                           # rescale exponent (combined) [tile parity][h] at 174 + 2 par + h
V_NMC = 178                          # n = -m c after half h, [h][rb] at 178 + 2 h + rb
V_NMCC = 182                         # n (combined) after the last half taken
V_SPAN, V_KSR = 183, 185             # [rb] row key range: length, start - 4 hh
V_MXA, V_MXB = 187, 189              # [rb] max-chain accumulators
V_M, V_D, V_MT = 191, 192, 193       # combined half max and running-max temporaries
V_NSENT = 194                        # n of the max sentinel
V_NINF = 195                         # -inf
V_RS = 196                           # 196..203 rescale temporaries
V_RA = 204                           # [rb] the exponent the rescale routine applies
V_MK = 206                           # 206..209 mask temporaries
V_LO = 210                           # [rb] mask: row start - 4 hh - first key of the tile
V_T = 188                            # epilogue temporaries (the loop's registers are free by then)
V_EPI = 209                          # 209..215 epilogue lane addresses
V_THR = 212                          # the row-sum check's threshold (loop only)
V_CHK = 213                          # row-sum check temporary (loop only)
V_LIMIT = 216                        # first VGPR left to the compiler

# clobbered SGPRs
S_RET = 52                  # return address of the rescale routine (2)
S_FLAG = 54                 # rescale flags [tile parity][h] (2 each) at 54 + 4 par + 2 h
S_T0, S_T1 = 62, 63
S_R1 = 64                   # r + 1 for step r (the tile whose scores the step computes)
S_N = 65                    # tile count
S_SPAN = 66                 # it1 - it0: tiles r + 1 - it0 below it need no range mask
S_KEY0 = 67                 # first key of tile r + 1 (masked steps)
S_KBYTES, S_VBYTES = 68, 69  # bytes from the current K / V^T descriptor base to the item's end
S_FORCE = 70                # nonzero: the next tile's half-0 check fails (2)
S_FORCE1 = 90               # nonzero: this tile's half-1 check fails (2)
S_KRS, S_VRS = 72, 76       # K / V^T buffer descriptors (4 each)
S_PAIRS = (80, 82, 84, 86)  # VALU compare results (2 each)
S_EIGHT, S_SENT = 88, 89    # 8.0 and the -2^30 max sentinel
S_FIRST, S_LASTC = 52, 91   # clobbered range

SENTINEL_BITS = 0xCE800000   # -2^30 as fp32 (V:174)
NEG_INF_BITS = 0xFF800000
EIGHT_BITS = 0x41000000
RSRC_WORD3 = 0x00020000
THR_BITS = 0x46000000        # 8192.0: a half passes its check when every lane's 16-key sum is at most this

TILE_BYTES = 16384           # one K or V^T tile in LDS
K_SLOTS = V_SLOTS = 4        # tile j+1's K and tile j's V^T are staged three steps before step j
V_RING = K_SLOTS * TILE_BYTES  # byte offset of the V^T ring
LDS_BYTES = V_RING + V_SLOTS * TILE_BYTES
EPI_REGION = 32 * 272 + 128  # per-wave O staging for 32 rows + their offsets
N_PRE_K, N_PRE_V = 4, 2      # operand reads of the next step issued before its barrier
PRO_LATE = 16                # prologue DMAs the pre step does not wait for

# ---------------------------------------------------------------------------
# instructions
# ---------------------------------------------------------------------------


def vreg(i, n=1):
    return f"v{i}" if n == 1 else f"v[{i}:{i + n - 1}]"


def areg(i, n=1):
    return f"a{i}" if n == 1 else f"a[{i}:{i + n - 1}]"


def sreg(i, n=1):
    return f"s{i}" if n == 1 else f"s[{i}:{i + n - 1}]"


def regs(f, i, n):
    return {f"{f}{i + k}" for k in range(n)}


class Ins:
    """One instruction with what the hazard and wait-count passes need."""

    def __init__(self, text, kind, rd=(), wr=(), *, trans=False, lgkm=False, vm=False,
                 mfma=None, mask_rd=(), branch=None, cond=False):
        self.text = text
        self.kind = kind          # mfma valu perm salu lds lds_w vmem_ld vmem_st dma nop wait barrier branch
        self.rd = set(rd)
        self.wr = set(wr)
        self.trans = trans
        self.lgkm = lgkm          # counted in lgkmcnt (LDS op)
        self.vm = vm              # counted in vmcnt
        self.mfma = mfma          # (dst_key, srcA regs, srcB regs, srcC regs or None)
        self.mask_rd = set(mask_rd)
        self.branch = branch      # target label
        self.cond = cond          # conditional branch (falls through too)
        self.urgent = False       # scheduled ahead of other ready work
        self.feeds_trans = False  # computes the input of an exponential


def mfma(dst, a, b, c_acc):
    """dst / a / b = (file, first); c_acc: True accumulates into dst, False
    starts from 0."""
    df, di = dst
    af, ai = a
    bf, bi = b
    dtxt = (vreg if df == "v" else areg)(di, 16)
    atxt = (vreg if af == "v" else areg)(ai, 4)
    btxt = (vreg if bf == "v" else areg)(bi, 4)
    ctxt = dtxt if c_acc else "0"
    dset = regs(df, di, 16)
    ab = regs(af, ai, 4) | regs(bf, bi, 4)
    rd = ab | (dset if c_acc else set())
    return Ins(f"v_mfma_f32_32x32x16_bf16 {dtxt}, {atxt}, {btxt}, {ctxt}", "mfma", rd, dset,
               mfma=((df, di), ab, dset if c_acc else None))


def valu(text, rd, wr, trans=False, mask_rd=()):
    return Ins(text, "valu", rd, wr, trans=trans, mask_rd=mask_rd)


def salu(text, rd=(), wr=()):
    return Ins(text, "salu", rd, wr)


def label(name):
    return Ins(f"{name}:", "label")


def branch(op, target, cond=True):
    return Ins(f"{op} {target}", "branch", branch=target, cond=cond)


def waitcnt(vm=None, lgkm=None):
    parts = []
    if vm is not None:
        parts.append(f"vmcnt({vm})")
    if lgkm is not None:
        parts.append(f"lgkmcnt({lgkm})")
    return Ins("s_waitcnt " + " ".join(parts), "wait")


# ---------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------


def s_in(name):
    return f"%[{name}]"


def kop(h, kk):
    return KOP_A + 4 * ((8 * h + kk) % K_SETS)


def k_read(h, kk, slot):
    """K operand of k-step kk for the 32 keys of half h of the tile in K
    slot `slot`."""
    dst = kop(h, kk)
    return Ins(f"ds_read_b128 {areg(dst, 4)}, {vreg(KOFF_V + kk)} offset:{slot * TILE_BYTES + h * 8192}",
               "lds", {f"v{KOFF_V + kk}"}, regs("a", dst, 4), lgkm=True)


def qk_mfmas(snxt, h, kk):
    return [mfma(("v", snxt + 32 * rb + 16 * h), ("a", kop(h, kk)), ("a", Q_A + 8 * kk + 4 * rb), kk > 0)
            for rb in range(2)]


def vop(s2, db):
    return VOP_A + 4 * ((4 * s2 + db) % V_SETS)


def v_read(s2, db, slot):
    """V^T operand (keys 16 s2.., head_dim block db) of the tile in V^T slot
    `slot` (the address registers include the ring's offset)."""
    dst = vop(s2, db)
    return Ins(f"ds_read_b128 {areg(dst, 4)}, {vreg(VOFF_V + s2)} offset:{slot * TILE_BYTES + db * 4096}",
               "lds", {f"v{VOFF_V + s2}"}, regs("a", dst, 4), lgkm=True)


def pv_mfmas(s2, db):
    return [mfma(("a", O_A + 32 * db + 16 * rb), ("a", vop(s2, db)), ("v", PK_V + 8 * s2 + 4 * rb), True)
            for rb in range(2)]


V_SEQ = [(s2, db) for s2 in range(4) for db in range(4)]


def dma(kind, i, slot):
    """One global -> LDS load of this wave's quarter of a K (kind 'k') or
    V^T tile into slot `slot` of its ring."""
    rs = S_KRS if kind == "k" else S_VRS
    base = slot * TILE_BYTES + (0 if kind == "k" else V_RING) + i * 1024
    off = s_in(f"{kind}dma{i}")
    return [salu(f"s_add_u32 m0, {s_in('ldsw')}, {base}", wr={"m0"}),
            Ins(f"buffer_load_dwordx4 {off}, {sreg(rs, 4)}, 0 offen lds", "dma",
                regs("s", rs, 4) | {"m0"}, set(), vm=True)]


def desc_advance(kind):
    """Move a descriptor on to the next tile: base += tile, the bytes left to
    the item's end shrink by a tile, and the record count is what is left
    (none past the item's last tile, part of the keys' last tile)."""
    if kind == "k":
        rs, nb, step = S_KRS, S_KBYTES, s_in("ktilebytes")
    else:
        rs, nb, step = S_VRS, S_VBYTES, str(TILE_BYTES)
    return [salu(f"s_add_u32 {sreg(rs)}, {sreg(rs)}, {step}"),
            salu(f"s_addc_u32 {sreg(rs + 1)}, {sreg(rs + 1)}, 0"),
            salu(f"s_sub_i32 {sreg(nb)}, {sreg(nb)}, {step}"),
            salu(f"s_max_i32 {sreg(rs + 2)}, {sreg(nb)}, 0")]


def half_elems(s, h):
    """The 32 registers of half h of the S tile at s, in packing order: for
    each pair (i, i+1) of a row block's 16 registers, row block 0 then 1."""
    out = []
    for i in range(0, 16, 2):
        for rb in range(2):
            base = s + 32 * rb + 16 * h
            out += [(rb, base + i), (rb, base + i + 1)]
    return out


def exps(s, h, lo, hi, nh=None):
    """P = 2^(s c + n) in place for elements lo..hi-1 of half h, with n the
    running -m c after half nh (default h) of the last tile whose max was
    taken."""
    out = []
    for rb, x in half_elems(s, h)[lo:hi]:
        nmc = V_NMC + 2 * (h if nh is None else nh) + rb
        out.append(valu(f"v_fma_f32 {vreg(x)}, {vreg(x)}, {s_in('c')}, {vreg(nmc)}",
                        {f"v{x}", f"v{nmc}"}, {f"v{x}"}))
        out[-1].feeds_trans = True
        out.append(valu(f"v_exp_f32 {vreg(x)}, {vreg(x)}", {f"v{x}"}, {f"v{x}"}, trans=True))
    return out


def packs(s, h):
    """P^T operands of half h packed to bf16: k-step s2 = 2 h + (i >= 8),
    register (i % 8) / 2 holds keys i, i+1 of the row block."""
    out = []
    for i in range(0, 16, 2):
        for rb in range(2):
            base = s + 32 * rb + 16 * h
            d = PK_V + 8 * (2 * h + (i >= 8)) + 4 * rb + (i % 8) // 2
            out.append(valu(f"v_cvt_pk_bf16_f32 {vreg(d)}, {vreg(base + i)}, {vreg(base + i + 1)}",
                            {f"v{base + i}", f"v{base + i + 1}"}, {f"v{d}"}))
    return out


def swap_combine(x, t, op):
    """x = op(x, x of the lane 32 apart) (v_permlane32_swap)."""
    return [valu(f"v_mov_b32 {vreg(t)}, {vreg(x)}", {f"v{x}"}, {f"v{t}"}),
            Ins(f"v_permlane32_swap_b32 {vreg(x)}, {vreg(t)}", "perm", {f"v{x}", f"v{t}"},
                {f"v{x}", f"v{t}"}),
            valu(f"{op} {vreg(x)}, {vreg(x)}, {vreg(t)}", {f"v{x}", f"v{t}"}, {f"v{x}"})]


def sums_tree(s, h):
    """This lane's sum of its 16 fp32 P of half h for each row block, in
    place (after the packing), left in the half's first register (the two
    lanes of a row keep partial sums of their own keys, combined once, at
    the end)."""
    return tree_levels(s, h, 16, 1)


def tree_levels(s, h, top, bottom):
    """The levels of sums_tree from `top` partial sums per row block down
    to `bottom` (16 -> 8 is the first level)."""
    out = []
    width = top
    while width > bottom:
        hw = width // 2
        for i in range(hw):
            for rb in range(2):
                b = s + 32 * rb + 16 * h
                out.append(valu(f"v_add_f32 {vreg(b + i)}, {vreg(b + i)}, {vreg(b + i + hw)}",
                                {f"v{b + i}", f"v{b + i + hw}"}, {f"v{b + i}"}))
        width = hw
    return out


def sums_add(s, h):
    """The half's lane sums (sums_tree) added to this lane's partial l."""
    out = []
    for rb in range(2):
        b = s + 32 * rb + 16 * h
        out.append(valu(f"v_add_f32 {vreg(V_L + rb)}, {vreg(V_L + rb)}, {vreg(b)}",
                        {f"v{V_L + rb}", f"v{b}"}, {f"v{V_L + rb}"}))
    return out


def running_max(s, h, par):
    """Row max of half h of S (per lane over its 16 keys, then the two lanes
    of each row with one lane swap that leaves the combined max: row block
    0 in lanes 0-31, row block 1 in lanes 32-63), then one running-max
    update for both row blocks: d = x c + n, the max moves when d > 8 (n
    becomes -x c and the rescale exponent is d, else 0), and the flag of
    (tile parity par, h) is set when some row moved from a finite max (a
    row still at the sentinel has O = 0 and l = 0); then n goes to each
    row block's lanes for the exponentials.  Marked urgent for the
    scheduler."""
    chains = []
    for rb in range(2):
        b = s + 32 * rb + 16 * h
        xa, xb = V_MXA + rb, V_MXB + rb
        c = [valu(f"v_max3_f32 {vreg(xa)}, {vreg(b)}, {vreg(b + 1)}, {vreg(b + 2)}", regs("v", b, 3), {f"v{xa}"}),
             valu(f"v_max3_f32 {vreg(xb)}, {vreg(b + 3)}, {vreg(b + 4)}, {vreg(b + 5)}", regs("v", b + 3, 3),
                  {f"v{xb}"})]
        acc = xa
        for i in range(6, 16, 2):
            c.append(valu(f"v_max3_f32 {vreg(acc)}, {vreg(acc)}, {vreg(b + i)}, {vreg(b + i + 1)}",
                          {f"v{acc}", f"v{b + i}", f"v{b + i + 1}"}, {f"v{acc}"}))
            acc = xb if acc == xa else xa
        c.append(valu(f"v_max_f32 {vreg(xa)}, {vreg(xa)}, {vreg(xb)}", {f"v{xa}", f"v{xb}"}, {f"v{xa}"}))
        chains.append(c)
    out = []
    for a, b in zip(chains[0], chains[1]):
        out += [a, b]
    x0, x1 = V_MXA, V_MXA + 1
    pm, pq = S_PAIRS[0], S_PAIRS[1]
    flag = S_FLAG + 4 * par + 2 * h
    al = V_AL + 2 * par + h
    n0, n1 = V_NMC + 2 * h, V_NMC + 2 * h + 1
    out += [
        Ins(f"v_permlane32_swap_b32 {vreg(x0)}, {vreg(x1)}", "perm", {f"v{x0}", f"v{x1}"}, {f"v{x0}", f"v{x1}"}),
        valu(f"v_max_f32 {vreg(V_M)}, {vreg(x0)}, {vreg(x1)}", {f"v{x0}", f"v{x1}"}, {f"v{V_M}"}),
        valu(f"v_fma_f32 {vreg(V_D)}, {vreg(V_M)}, {s_in('c')}, {vreg(V_NMCC)}", {f"v{V_M}", f"v{V_NMCC}"},
             {f"v{V_D}"}),
        valu(f"v_cmp_neq_f32_e64 {sreg(pq, 2)}, {vreg(V_NSENT)}, {vreg(V_NMCC)}", {f"v{V_NSENT}", f"v{V_NMCC}"},
             {f"s{pq}", f"s{pq + 1}"}),
        valu(f"v_mul_f32 {vreg(V_MT)}, {s_in('negc')}, {vreg(V_M)}", {f"v{V_M}"}, {f"v{V_MT}"}),
        valu(f"v_cmp_lt_f32_e64 {sreg(pm, 2)}, {sreg(S_EIGHT)}, {vreg(V_D)}", {f"v{V_D}", f"s{S_EIGHT}"},
             {f"s{pm}", f"s{pm + 1}"}),
        valu(f"v_cndmask_b32_e64 {vreg(al)}, 0, {vreg(V_D)}, {sreg(pm, 2)}", {f"v{V_D}"}, {f"v{al}"},
             mask_rd={f"s{pm}", f"s{pm + 1}"}),
        valu(f"v_cndmask_b32_e64 {vreg(V_NMCC)}, {vreg(V_NMCC)}, {vreg(V_MT)}, {sreg(pm, 2)}",
             {f"v{V_NMCC}", f"v{V_MT}"}, {f"v{V_NMCC}"}, mask_rd={f"s{pm}", f"s{pm + 1}"}),
        salu(f"s_and_b64 {sreg(flag, 2)}, {sreg(pq, 2)}, {sreg(pm, 2)}",
             {f"s{pq}", f"s{pq + 1}", f"s{pm}", f"s{pm + 1}"}, {f"s{flag}", f"s{flag + 1}"}),
        valu(f"v_mov_b32 {vreg(n0)}, {vreg(V_NMCC)}", {f"v{V_NMCC}"}, {f"v{n0}"}),
        valu(f"v_mov_b32 {vreg(n1)}, {vreg(V_NMCC)}", {f"v{V_NMCC}"}, {f"v{n1}"}),
        Ins(f"v_permlane32_swap_b32 {vreg(n0)}, {vreg(n1)}", "perm", {f"v{n0}", f"v{n1}"}, {f"v{n0}", f"v{n1}"}),
    ]
    for x in out:
        x.urgent = True
    return out


def mask(s, h, key0=S_KEY0):
    """Scores of half h outside each row's [start, end) set to -inf.
    Register r of the half is key 32 h + 8 (r >> 2) + 4 hh + (r & 3) of the
    tile; the row bounds were shifted by 4 hh, so it is legal iff
    (off - lo) < span, unsigned, with lo = start - 4 hh - key0 (the tile's
    first key, in SGPR key0)."""
    out = []
    for rb in range(2):
        out.append(valu(f"v_subrev_u32 {vreg(V_LO + rb)}, {sreg(key0)}, {vreg(V_KSR + rb)}",
                        {f"v{V_KSR + rb}", f"s{key0}"}, {f"v{V_LO + rb}"}))
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


def rescale_routine():
    """alpha = 2^-e for the rescale exponent e of each row (v[V_RA + rb],
    0 for rows whose max did not move), then l *= alpha and O *= alpha;
    entered by a branch with the return address in S_RET."""
    out = []
    for rb in range(2):
        r = V_RA + rb
        out.append(valu(f"v_exp_f32_e64 {vreg(r)}, -{vreg(r)}", {f"v{r}"}, {f"v{r}"}, trans=True))
    for rb in range(2):
        out.append(valu(f"v_mul_f32 {vreg(V_L + rb)}, {vreg(V_L + rb)}, {vreg(V_RA + rb)}",
                        {f"v{V_L + rb}", f"v{V_RA + rb}"}, {f"v{V_L + rb}"}))
    for rb in range(2):
        for db in range(4):
            for half in range(2):
                base = O_A + 32 * db + 16 * rb + 8 * half
                for k in range(8):
                    out.append(valu(f"v_accvgpr_read_b32 {vreg(V_RS + k)}, {areg(base + k)}", {f"a{base + k}"},
                                    {f"v{V_RS + k}"}))
                for k in range(8):
                    out.append(valu(f"v_mul_f32 {vreg(V_RS + k)}, {vreg(V_RS + k)}, {vreg(V_RA + rb)}",
                                    {f"v{V_RS + k}", f"v{V_RA + rb}"}, {f"v{V_RS + k}"}))
                for k in range(8):
                    out.append(valu(f"v_accvgpr_write_b32 {areg(base + k)}, {vreg(V_RS + k)}", {f"v{V_RS + k}"},
                                    {f"a{base + k}"}))
    out.append(Ins(f"s_setpc_b64 {sreg(S_RET, 2)}", "ret"))
    return out


# ---------------------------------------------------------------------------
# list scheduling of a block
# ---------------------------------------------------------------------------

MF_DIST = 12          # instructions between an MFMA and a VALU read of its result


def _conflict(a, b):
    """b must stay after a (program order) if they touch a common register
    with at least one write."""
    return bool(a.wr & (b.rd | b.wr | b.mask_rd) or b.wr & (a.rd | a.mask_rd))


def _dist(a, b):
    """Instructions b must trail a by (a before b, conflicting): the
    wait states gfx950 needs between them, so that no s_nop is needed."""
    if a.trans and a.wr & (b.rd | b.mask_rd):
        return 3
    if b.kind == "perm" and a.wr & b.rd:
        return 3
    if any(r.startswith("s") for r in a.wr & b.mask_rd) and a.kind != "salu":
        return 3
    return 1


def schedule(mfmas, valu_list, side=None, carry=False, n_carried=0, lead_cap=2, one_feed=False):
    """Order one block: the MFMAs in their given order, side(i) (LDS reads,
    DMAs, descriptor updates) right before MFMA i and side(len) after the
    last, and the VALU / SALU list (in a valid program order) spread over
    the gaps between MFMAs (slot s: before MFMA s) so that every gap issues
    about the same number of instructions, side work included (a wave
    issues about one instruction per five to six cycles, so the gaps are
    where the MFMAs wait).  Work that touches an MFMA's registers stays
    after that MFMA (MF_DIST instructions after it for a read of its
    result), and work that touches a side instruction's registers stays
    after it; the first n_carried items come from the previous block
    instead and go before any MFMA of this block whose registers they
    touch.  Dependent instructions keep the distance gfx950 needs between
    them.  Each gap takes at most one exponential, never as its first
    instruction; exponentials (and the FMAs that feed them), then urgent
    work, go first among what is ready.  With one_feed, a gap also takes at
    most one instruction that feeds an exponential, so that the feeding
    work keeps pace with the exponentials and can open the next gaps.  With
    carry, what does not fit is returned for the next block instead of
    being issued after the last MFMA."""
    n = len(valu_list)
    nm = len(mfmas)
    sides = [side(i) if side is not None else [] for i in range(nm + 1)]
    preds = [[] for _ in range(n)]
    for j in range(n):
        for i in range(j):
            if _conflict(valu_list[i], valu_list[j]):
                preds[j].append(i)
    succs = [[] for _ in range(n)]
    for j in range(n):
        for i in preds[j]:
            succs[i].append(j)
    min_slot = [0] * n
    deadline = [nm] * n
    mf_users = [[] for _ in range(nm)]
    for j, v in enumerate(valu_list):
        for i, m in enumerate(mfmas):
            if _conflict(m, v):
                if j < n_carried:
                    deadline[j] = min(deadline[j], i)
                else:
                    min_slot[j] = max(min_slot[j], i + 1)
                    if m.wr & (v.rd | v.wr | v.mask_rd):
                        mf_users[i].append(j)
        for i in range(nm):
            if any(_conflict(x, v) for x in sides[i]):
                assert j >= n_carried or deadline[j] == nm
                min_slot[j] = max(min_slot[j], i + 1)
        if any(_conflict(x, v) for x in sides[nm]):
            assert not carry, "a carried instruction conflicts with the block's last side work"
    for j in reversed(range(n)):      # successors first: deadlines pass down whole chains
        for k in preds[j]:
            deadline[k] = min(deadline[k], deadline[j])
    issued = [False] * n
    npred = [len(p) for p in preds]
    ready = [0] * n
    out = []
    st = {"pos": 0, "fed": 0, "done": 0}

    def put(x):
        out.append(x)
        st["pos"] += 1

    def issue(j):
        issued[j] = True
        v = valu_list[j]
        put(v)
        if v.feeds_trans:
            st["fed"] += 1
        if v.trans and st["fed"]:
            st["fed"] -= 1
        for k in succs[j]:
            npred[k] -= 1
            ready[k] = max(ready[k], st["pos"] - 1 + _dist(v, valu_list[k]))
        st["done"] += 1

    def pick(slot, first, n_exp, n_feed=0, relax=False):
        best = None
        for j in range(n):
            if issued[j] or npred[j] or min_slot[j] > slot or (ready[j] > st["pos"] and not relax):
                continue
            v = valu_list[j]
            if v.trans and (first or n_exp >= 1) and not relax:
                continue
            if one_feed and v.feeds_trans and n_feed >= 1 and not relax:
                continue
            lead = v.trans or (v.feeds_trans and st["fed"] < 2)
            key = (not lead, not v.urgent, j)
            if best is None or key < best[1]:
                best = (j, key)
        return None if best is None else best[0]

    def fill(slot, cap, drain=False):
        first, n_exp, n_feed, cnt = True, 0, 0, 0
        while cnt < cap:
            j = pick(slot, first, n_exp, n_feed)
            if j is None and drain:
                j = pick(slot, first, n_exp, n_feed, relax=True)
            if j is None:
                break
            issue(j)
            first = False
            n_exp += valu_list[j].trans
            n_feed += valu_list[j].feeds_trans
            cnt += 1

    def force(i):
        """Issue, in list order, the carried work MFMA i must follow."""
        for j in range(n):
            if not issued[j] and deadline[j] <= i:
                assert npred[j] == 0
                issue(j)

    side_left = sum(len(s) for s in sides)
    for i in range(nm + 1):
        remaining = n - st["done"] + side_left
        if i == 0:
            cap = lead_cap if nm else n
        elif i == nm and not carry:
            cap = n
        else:
            cap = max(1, -(-remaining // (nm + 1 - i)) - len(sides[i]))
        # an M0 write goes ahead of the slot's VALU work: the LDS DMA after
        # it then needs no s_nop
        early = [x for x in sides[i] if "m0" in x.wr]
        assert len(early) <= 1
        for x in early:
            put(x)
        fill(i, cap, drain=(i == nm and not carry) or not nm)
        for x in sides[i]:
            if x not in early:
                put(x)
        side_left -= len(sides[i])
        if i < nm:
            force(i)
            put(mfmas[i])
            for j in mf_users[i]:
                ready[j] = max(ready[j], st["pos"] - 1 + MF_DIST)
    left = [valu_list[j] for j in range(n) if not issued[j]]
    if not carry or not nm:
        assert not left, "unscheduled work"
    return out, left


# ---------------------------------------------------------------------------
# blocks of a step
# ---------------------------------------------------------------------------
# Step r (phase q = r mod 4) computes S(r+1) from K(r+1) in K slot (q+1)%4
# and P(r) V(r) from V^T(r) in V^T slot q; it stages K(r+4) into K slot q
# (read by step r-1) and V^T(r+3) into V^T slot (q+3)%4 (read by step r-1),
# and at its end reads the first operands of K(r+2) and V^T(r+1).

def split_left(left, regs_):
    """Leftover work of a block before a check: what touches regs_ (or must
    precede such work) is issued at the block's end, the rest is carried
    on.  Both lists keep their program order."""
    must = [bool((x.rd | x.wr | x.mask_rd) & regs_) for x in left]
    for j in reversed(range(len(left))):
        if must[j]:
            for i in range(j):
                if not must[i] and _conflict(left[i], left[j]):
                    must[i] = True
    return [x for x, m in zip(left, must) if m], [x for x, m in zip(left, must) if not m]


def half_regs(s, h):
    """The S / P registers of half h of the tile at s, and its P^T operands."""
    r = {f"v{s + 32 * rb + 16 * h + i}" for rb in range(2) for i in range(16)}
    return r | regs("v", PK_V + 16 * h, 16)


# the temporaries of mask() and the row sums a recomputation also writes
CHECK_TEMPS = ({f"v{V_L}", f"v{V_L + 1}", f"v{V_CHK}", "vcc"} | regs("v", V_LO, 2) | regs("v", V_MK, 4) |
               regs("s", S_PAIRS[0], 8) | regs("s", S_T0, 2))


def block_a(q, kind, masked, opt=False):
    """S(j+1) = K(j+1) Q^T in 32 MFMAs (half 0, then half 1).  A step
    starts with P(j) half 0 exponentiated, packed and its sums' first level
    formed, and the first 16 exponentials of P(j) half 1 taken (by the
    previous step's B2).  A takes the last 16 exponentials of P(j) half 1
    and the rest of half 0's sums (and, with opt, half 0's check); once
    S(j+1) half 0 is final, its mask, (without opt) its running max, and
    its first 16 exponentials; then P(j) half 1 is packed and its sums
    formed, work that may carry on into B1 (with opt, what is left of half
    0 is issued before the check instead).  kind 'pre' (tile 0's S and the
    work a step starts with), 'full', 'last' (no S(j+1)).  Returns
    (instructions, leftover VALU)."""
    par = q % 2
    scur, snxt = S_V[par], S_V[1 - par]
    pn = 1 - par           # parity of tile j + 1
    ks = (q + 1) % 4
    nh = 1 if opt else None
    out = []
    vl = []
    if kind != "pre":
        vl += exps(scur, 1, 16, 32) + tree_levels(scur, 0, 8, 1)
        if opt:
            vl += check_items(par, 0)
    if kind != "last":
        if masked:
            out += [salu(f"s_lshl_b32 {sreg(S_KEY0)}, {sreg(S_R1)}, 6"),
                    salu(f"s_add_u32 {sreg(S_KEY0)}, {sreg(S_KEY0)}, {s_in('key0')}")]
            vl += mask(snxt, 0)
        if not opt:
            vl += running_max(snxt, 0, pn)
        vl += exps(snxt, 0, 0, 16 if kind != "pre" else 32, nh)
    if kind != "pre":
        vl += packs(scur, 1) + sums_tree(scur, 1)
    if kind == "last":
        out += [v_read(*x, q) for x in V_SEQ[N_PRE_V:V_SETS - 1]]
        o, _ = schedule([], vl)
        return out + o, []
    dmas = [dma("k", i, q) for i in range(4)]
    mf = []
    for h in range(2):
        for kk in range(8):
            mf += qk_mfmas(snxt, h, kk)
    reads = [(h, kk) for h in range(2) for kk in range(8)]
    pre = N_PRE_K if kind != "pre" else 0     # K operands read before the barrier
    vre = [V_SEQ[k] for k in range(N_PRE_V, V_SETS - 1)] if kind == "full" else []

    def side(i):
        r = []
        if i == 0:
            r += [k_read(*x, ks) for x in reads[pre:6]]
        qq = i // 2
        if i % 2 == 1 and qq + 6 < 16:
            r.append(k_read(*reads[qq + 6], ks))
        if i % 8 == 4:
            r += dmas[i // 8]
            if i // 8 == 3:
                r += desc_advance("k")
        if vre and i >= 26 and i % 2 == 0 and (i - 26) // 2 < len(vre):
            r.append(v_read(*vre[(i - 26) // 2], q))
        return r
    o, left = schedule(mf, vl, side, carry=True)
    if opt:
        must, left = split_left(left, half_regs(scur, 0) | CHECK_TEMPS)
        o += must
    return out + o, left


def block_b1(q, kind, masked, carried, opt=False):
    """P(j) V(j) for half 0 (16 MFMAs) while P(j) half 0's sums are added
    to l, S(j+1) half 0 takes its last 16 exponentials, S(j+1) half 1 is
    masked and (without opt) given its running max, and P(j) half 1's
    packing and sums carried from A finish (with opt, with its check; what
    is left of half 1 is then issued before the check, the exponentials
    carry on).  kind 'pre': the V^T copies of the pre step only.  Returns
    (instructions, leftover VALU)."""
    par = q % 2
    snxt, scur = S_V[1 - par], S_V[par]
    pn = 1 - par
    nh = 1 if opt else None
    vl = list(carried)
    nc = len(vl)
    if kind != "pre":
        vl += sums_add(scur, 0)
    if kind == "full":
        vl += exps(snxt, 0, 16, 32, nh)
    if kind != "last":
        if masked:
            vl += mask(snxt, 1)
        if not opt:
            vl += running_max(snxt, 1, pn)
    if opt and kind != "pre":
        vl += check_items(par, 1)
    dmas = [dma("v", i, (q + 3) % 4) for i in range(4)] if kind != "last" else []
    if kind == "pre":
        o, _ = schedule([], vl)
        for d in dmas:
            o += d
        return o + desc_advance("v"), []
    mf = []
    for s2 in (0, 1):
        for db in range(4):
            mf += pv_mfmas(s2, db)

    def side(i):
        r = []
        qq = i // 2
        if i % 2 == 1 and qq + V_SETS - 1 < 16:
            r.append(v_read(*V_SEQ[qq + V_SETS - 1], q))
        if i % 4 == 2 and dmas:
            r += dmas[i // 4]
            if i // 4 == 3:
                r += desc_advance("v")
        return r
    o, left = schedule(mf, vl, side, carry=True, n_carried=nc, lead_cap=0)
    must, left = split_left(left, (half_regs(scur, 1) | CHECK_TEMPS) if opt else {f"v{V_L}", f"v{V_L + 1}"})
    o += must
    return o, left


def block_b2(q, kind, carried, opt=False):
    """P(j) V(j) for half 1 (16 MFMAs) while P(j) half 1's sums are added
    to l and S(j+1) half 1 takes its first 16 exponentials, S(j+1) half 0
    is packed and its sums' first level formed (the state the next step
    starts with); then the next step's first K(j+2) and V^T(j+1) operands
    are read.  kind 'pre': S(0) half 1's first 16 exponentials, S(0) half
    0's packing and first level, then the pre step's own barrier."""
    par = q % 2
    scur, snxt = S_V[par], S_V[1 - par]
    nh = 1 if opt else None
    vl = list(carried)
    nc = len(vl)
    if kind != "pre":
        vl += sums_add(scur, 1)
    if kind != "last":
        vl += exps(snxt, 1, 0, 16, nh) + packs(snxt, 0) + tree_levels(snxt, 0, 16, 8)
    mf = []
    if kind != "pre":
        for s2 in (2, 3):
            for db in range(4):
                mf += pv_mfmas(s2, db)

    def side(i):
        if i == len(mf):
            if kind == "last":
                return []
            # the pre step's own barrier: K(1) and V^T(0) have landed in
            # every wave before they are read
            sync = [waitcnt(vm=PRO_LATE), Ins("s_barrier", "barrier")] if kind == "pre" else []
            return sync + ([k_read(0, kk, (q + 2) % 4) for kk in range(N_PRE_K)] +
                           [v_read(*V_SEQ[k], (q + 1) % 4) for k in range(N_PRE_V)])
        qq = 8 + i // 2
        if i % 2 == 1 and qq + V_SETS - 1 < 16:
            return [v_read(*V_SEQ[qq + V_SETS - 1], q)]
        return []
    o, _ = schedule(mf, vl, side, n_carried=nc, lead_cap=2)
    return o


# ---------------------------------------------------------------------------


class Block:
    def __init__(self, name, ins, ret_point=False):
        self.name = name
        self.ins = ins
        self.ret_point = ret_point    # the rescale routine may return here


COLD = []     # out-of-line call blocks, laid out after the loop


def _cold_call(tag, skip, target, prep=()):
    """An out-of-line block that drains the LDS reads, sets the return
    address to `skip` and branches to the routine at `target`.  The block
    is laid out after `skip` (program() places COLD after every step), so
    the return address is the program counter minus a positive distance
    (a 64-bit subtraction: adding the negative 32-bit difference with a
    carry into the high word would be off by 2^32); generate() checks the
    order."""
    u = "%="
    pc = f"L{tag}_pc_{u}"
    COLD.append(Block(f"L{tag}_c_{u}", list(prep) + [
        waitcnt(lgkm=0),
        Ins(f"s_getpc_b64 {sreg(S_RET, 2)}", "salu", set(), {f"s{S_RET}", f"s{S_RET + 1}"}),
        label(pc),
        salu(f"s_sub_u32 {sreg(S_RET)}, {sreg(S_RET)}, {pc}-{skip}"),
        salu(f"s_subb_u32 {sreg(S_RET + 1)}, {sreg(S_RET + 1)}, 0"),
        Ins(f"s_branch {target}", "call", branch=target, cond=False),
    ]))
    return f"L{tag}_c_{u}"


def check_returns(blocks):
    """A return address formed as pc - (pc - skip) needs the skip label
    before the call's pc label in the layout, one formed as pc + (ret - pc)
    (the 32-bit difference with a carry into the high word) the return
    label after it."""
    pos = {}
    n = 0
    for b in blocks:
        pos[b.name] = n
        for ins in b.ins:
            n += 1
            if ins.kind == "label":
                pos[ins.text[:-1]] = n
    for b in blocks:
        for ins in b.ins:
            if ins.text.startswith(f"s_sub_u32 {sreg(S_RET)}, {sreg(S_RET)}, "):
                pc, skip = ins.text.split(", ")[-1].split("-")
                assert pos[skip] < pos[pc], f"return label {skip} after its call"
            if ins.text.startswith(f"s_add_u32 {sreg(S_RET)}, {sreg(S_RET)}, "):
                ret, pc = ins.text.split(", ")[-1].split("-")
                assert pos[ret] > pos[pc], f"return label {ret} before its call"


def call_rescale(tag, par, h):
    """Blocks that apply O, l *= 2^-e(tile of parity par, half h) when that
    tile half's flag is set: test (and clear) the flag, then (rarely, out
    of line) give each row block its exponents, drain the LDS reads and
    branch to the shared routine with the return address."""
    u = "%="
    flag = S_FLAG + 4 * par + 2 * h
    skip = f"L{tag}_x_{u}"
    al = V_AL + 2 * par + h
    call = _cold_call(tag, skip, f"Lrescale_{u}", [
        valu(f"v_mov_b32 {vreg(V_RA)}, {vreg(al)}", {f"v{al}"}, {f"v{V_RA}"}),
        valu(f"v_mov_b32 {vreg(V_RA + 1)}, {vreg(al)}", {f"v{al}"}, {f"v{V_RA + 1}"}),
        Ins(f"v_permlane32_swap_b32 {vreg(V_RA)}, {vreg(V_RA + 1)}", "perm", {f"v{V_RA}", f"v{V_RA + 1}"},
            {f"v{V_RA}", f"v{V_RA + 1}"})])
    # the flag is cleared once tested: steps that take no running max leave
    # it clear unless a recomputation sets it
    test = Block(f"L{tag}_t_{u}", [salu(f"s_cmp_lg_u64 {sreg(flag, 2)}, 0"),
                                   salu(f"s_mov_b64 {sreg(flag, 2)}, 0", wr={f"s{flag}", f"s{flag + 1}"}),
                                   branch("s_cbranch_scc1", call)])
    return [test, Block(skip, [], ret_point=True)]


def call_recompute(tag, par, h, head):
    """Blocks that end `head` with the test that check_items left: nothing
    to do unless half h of tile j (parity par) failed its check or its
    rescale flag is set.  Then, out of line: the recomputation if the check
    failed (its routine returns into the out-of-line blocks), and the O, l
    rescale if the flag is set (then cleared), with the LDS reads drained
    before each branch to a shared routine; back to the step after."""
    u = "%="
    skip = f"L{tag}_x_{u}"
    pr = S_T0
    flag = S_FLAG + 4 * par + 2 * h
    al = V_AL + 2 * par + h
    cold, resc, back = f"L{tag}_o_{u}", f"L{tag}_r_{u}", f"L{tag}_b_{u}"
    pc0, pc1 = f"L{tag}_pc_{u}", f"L{tag}_pd_{u}"
    COLD.extend([
        Block(cold, [salu("s_cmp_lg_u64 vcc, 0", {"vcc"}), branch("s_cbranch_scc0", resc)]),
        Block(f"L{tag}_c_{u}", [
            waitcnt(lgkm=0),
            Ins(f"s_getpc_b64 {sreg(S_RET, 2)}", "salu", set(), {f"s{S_RET}", f"s{S_RET + 1}"}),
            label(pc0),
            salu(f"s_add_u32 {sreg(S_RET)}, {sreg(S_RET)}, {resc}-{pc0}"),
            salu(f"s_addc_u32 {sreg(S_RET + 1)}, {sreg(S_RET + 1)}, 0"),
            Ins(f"s_branch Lrecomp{par}{h}_{u}", "call", branch=f"Lrecomp{par}{h}_{u}", cond=False)]),
        Block(resc, [salu(f"s_cmp_lg_u64 {sreg(flag, 2)}, 0"),
                     salu(f"s_mov_b64 {sreg(flag, 2)}, 0", wr={f"s{flag}", f"s{flag + 1}"}),
                     branch("s_cbranch_scc0", back)], ret_point=True),
        Block(f"L{tag}_s_{u}", [
            valu(f"v_mov_b32 {vreg(V_RA)}, {vreg(al)}", {f"v{al}"}, {f"v{V_RA}"}),
            valu(f"v_mov_b32 {vreg(V_RA + 1)}, {vreg(al)}", {f"v{al}"}, {f"v{V_RA + 1}"}),
            Ins(f"v_permlane32_swap_b32 {vreg(V_RA)}, {vreg(V_RA + 1)}", "perm", {f"v{V_RA}", f"v{V_RA + 1}"},
                {f"v{V_RA}", f"v{V_RA + 1}"}),
            waitcnt(lgkm=0),
            Ins(f"s_getpc_b64 {sreg(S_RET, 2)}", "salu", set(), {f"s{S_RET}", f"s{S_RET + 1}"}),
            label(pc1),
            salu(f"s_sub_u32 {sreg(S_RET)}, {sreg(S_RET)}, {pc1}-{skip}"),
            salu(f"s_subb_u32 {sreg(S_RET + 1)}, {sreg(S_RET + 1)}, 0"),
            Ins(f"s_branch Lrescale_{u}", "call", branch=f"Lrescale_{u}", cond=False)]),
        Block(back, [branch("s_branch", skip, cond=False)]),
    ])
    chk = [salu(f"s_cmp_lg_u64 {sreg(pr, 2)}, 0", {f"s{pr}", f"s{pr + 1}"}), branch("s_cbranch_scc1", cold)]
    return [Block(f"L{tag}_k_{u}", head + chk), Block(skip, [], ret_point=True)]


def check_items(par, h):
    """The test of half h of tile j (parity par) that call_recompute
    branches on, as ordinary work for the scheduler: vcc = lanes whose
    16-key sum of either row block (left by sums_tree) exceeds the
    threshold, or every lane when a recomputation is forced; s[S_T0:S_T0+1]
    = vcc or the half's rescale flag (steps without a running max set that
    flag only by recomputing, after this test, or in step 0 for tile 1,
    before it)."""
    s = S_V[par]
    pr = S_T0
    force = S_FORCE if h == 0 else S_FORCE1
    flag = S_FLAG + 4 * par + 2 * h
    return [valu(f"v_max_f32 {vreg(V_CHK)}, {vreg(s + 16 * h)}, {vreg(s + 32 + 16 * h)}",
                 {f"v{s + 16 * h}", f"v{s + 32 + 16 * h}"}, {f"v{V_CHK}"}),
            valu(f"v_cmp_lt_f32_e64 vcc, {vreg(V_THR)}, {vreg(V_CHK)}", {f"v{V_THR}", f"v{V_CHK}"}, {"vcc"}),
            # mask_rd: keeps the scalar read three instructions after the compare
            Ins(f"s_or_b64 vcc, vcc, {sreg(force, 2)}", "salu", {f"s{force}", f"s{force + 1}"}, {"vcc"},
                mask_rd={"vcc"}),
            salu(f"s_or_b64 {sreg(pr, 2)}, vcc, {sreg(flag, 2)}", {"vcc", f"s{flag}", f"s{flag + 1}"},
                 {f"s{pr}", f"s{pr + 1}"})]


def recompute_routine(par, h):
    """Half h of tile j = r of step r (S_R1 - 1; scores in S buffer par)
    failed its check: its exponentials may exceed the threshold or be
    infinite, or (half 1) the max moved in half 0 after they were taken.
    Its K rows come straight from memory (the LDS slot is being refilled);
    the half's scores are recomputed by the same MFMAs in the same order,
    masked, given the exact running max (O, l *= 2^-e then follows at the
    step's rescale point), exponentiated, packed and summed as the step
    would have.  Where a row's max moved from a finite value, the
    exponentials taken since with the old max are redone too: half 0 forces
    half 1's check, half 1 the next tile's half-0 check.  Entered by a
    branch with the return address in S_RET."""
    s = S_V[par]
    rs, t0, t1 = S_PAIRS[2], S_T0, S_T1
    o0, lane = V_RS, s_in("lane")
    out = [salu(f"s_sub_u32 {sreg(t0)}, {sreg(S_R1)}, 1", {f"s{S_R1}"}, {f"s{t0}"}),
           salu(f"s_mul_i32 {sreg(t0)}, {sreg(t0)}, {s_in('ktilebytes')}", {f"s{t0}"}, {f"s{t0}"}),
           salu(f"s_mov_b64 {sreg(rs, 2)}, {s_in('kbase')}", set(), {f"s{rs}", f"s{rs + 1}"}),
           salu(f"s_add_u32 {sreg(rs)}, {sreg(rs)}, {sreg(t0)}", {f"s{rs}", f"s{t0}"}, {f"s{rs}"}),
           salu(f"s_addc_u32 {sreg(rs + 1)}, {sreg(rs + 1)}, 0", {f"s{rs + 1}"}, {f"s{rs + 1}"}),
           salu(f"s_sub_i32 {sreg(rs + 2)}, {s_in('kbytes')}, {sreg(t0)}", {f"s{t0}"}, {f"s{rs + 2}"}),
           salu(f"s_max_i32 {sreg(rs + 2)}, {sreg(rs + 2)}, 0", {f"s{rs + 2}"}, {f"s{rs + 2}"}),
           salu(f"s_mov_b32 {sreg(rs + 3)}, {RSRC_WORD3:#x}", set(), {f"s{rs + 3}"}),
           salu(f"s_lshr_b32 {sreg(t1)}, {s_in('ktilebytes')}, 6", set(), {f"s{t1}"}),
           # lane l loads key 32 h + (l & 31), head_dim 8 (l >> 5) + 16 kk
           valu(f"v_and_b32 {vreg(o0)}, 31, {lane}", set(), {f"v{o0}"}),
           valu(f"v_add_u32 {vreg(o0)}, {32 * h}, {vreg(o0)}", {f"v{o0}"}, {f"v{o0}"}),
           valu(f"v_mul_u32_u24 {vreg(o0)}, {sreg(t1)}, {vreg(o0)}", {f"v{o0}", f"s{t1}"}, {f"v{o0}"}),
           valu(f"v_lshrrev_b32 {vreg(o0 + 1)}, 5, {lane}", set(), {f"v{o0 + 1}"}),
           valu(f"v_lshl_add_u32 {vreg(o0)}, {vreg(o0 + 1)}, 4, {vreg(o0)}", {f"v{o0}", f"v{o0 + 1}"},
                {f"v{o0}"})]
    for kk in range(8):
        d = KOP_A + 4 * kk
        out.append(Ins(f"buffer_load_dwordx4 {areg(d, 4)}, {vreg(o0)}, {sreg(rs, 4)}, 0 offen offset:{32 * kk}",
                       "vmem_ld", {f"v{o0}"} | regs("s", rs, 4), regs("a", d, 4), vm=True))
    out.append(waitcnt(vm=0))
    for kk in range(8):
        for rb in range(2):
            out.append(mfma(("v", s + 32 * rb + 16 * h), ("a", KOP_A + 4 * kk), ("a", Q_A + 8 * kk + 4 * rb),
                            kk > 0))
    out += [salu(f"s_sub_u32 {sreg(t0)}, {sreg(S_R1)}, 1", {f"s{S_R1}"}, {f"s{t0}"}),
            salu(f"s_lshl_b32 {sreg(t0)}, {sreg(t0)}, 6", {f"s{t0}"}, {f"s{t0}"}),
            salu(f"s_add_u32 {sreg(t0)}, {sreg(t0)}, {s_in('key0')}", {f"s{t0}"}, {f"s{t0}"})]
    vl = mask(s, h, key0=t0) + running_max(s, h, par) + exps(s, h, 0, 32) + packs(s, h) + sums_tree(s, h)
    if h == 0:
        # the steps without a running max exponentiate with n after half 1
        vl += [valu(f"v_mov_b32 {vreg(V_NMC + 2 + rb)}, {vreg(V_NMC + rb)}", {f"v{V_NMC + rb}"},
                    {f"v{V_NMC + 2 + rb}"}) for rb in range(2)]
    o, _ = schedule([], vl)
    out += o
    flag = S_FLAG + 4 * par + 2 * h
    if h == 0:
        # half 1 of this tile and the first exponentials of the next tile's
        # half 0 were taken with the old max
        out += [salu(f"s_mov_b64 {sreg(S_FORCE1, 2)}, {sreg(flag, 2)}", {f"s{flag}", f"s{flag + 1}"},
                     {f"s{S_FORCE1}", f"s{S_FORCE1 + 1}"}),
                salu(f"s_mov_b64 {sreg(S_FORCE, 2)}, {sreg(flag, 2)}", {f"s{flag}", f"s{flag + 1}"},
                     {f"s{S_FORCE}", f"s{S_FORCE + 1}"})]
    else:
        out += [salu(f"s_or_b64 {sreg(S_FORCE, 2)}, {sreg(S_FORCE, 2)}, {sreg(flag, 2)}",
                     {f"s{flag}", f"s{flag + 1}", f"s{S_FORCE}", f"s{S_FORCE + 1}"},
                     {f"s{S_FORCE}", f"s{S_FORCE + 1}"}),
                salu(f"s_mov_b64 {sreg(S_FORCE1, 2)}, 0", set(), {f"s{S_FORCE1}", f"s{S_FORCE1 + 1}"})]
    out += [Ins("s_nop 15", "nop"), Ins(f"s_setpc_b64 {sreg(S_RET, 2)}", "ret")]
    return out


def opt_tail(tag, q, kind, masked):
    """A step without running max: its A block and the check of P(j) half
    0, O, l *= 2^-e(j, 0) if needed, B1 and the check of P(j) half 1, O, l
    *= 2^-e(j, 1) if needed, B2 (work left over by one block carried into
    the next)."""
    u = "%="
    par = q % 2
    a, left = block_a(q, kind, masked, opt=True)
    bl = call_recompute(f"{tag}k0", par, 0, a)
    b1, left = block_b1(q, kind, masked, left, opt=True)
    bl += call_recompute(f"{tag}k1", par, 1, b1)
    bl.append(Block(f"L{tag}_b2_{u}", block_b2(q, kind, left, opt=True)))
    return bl


def step_blocks(tag, q, kind, end_label, opt=True):
    """kind: 'pre' (S of the first tile only), 'full', 'last' (P V only).
    A full step with the running max (opt False): wait and barrier, O, l *=
    2^-e(j, 0) if needed, then an unmasked or a masked copy of A, B1, O, l
    *= 2^-e(j, 1) if needed, B2.  Without it (opt): wait and barrier, then
    an unmasked or a masked copy of A and opt_tail."""
    u = "%="
    par = q % 2
    blocks = []
    if kind == "pre":
        # the first tile always takes the range mask (a no-op where all its
        # keys are legal)
        a, left = block_a(q, "pre", True)
        b1, left = block_b1(q, "pre", True, left)
        b2 = block_b2(q, "pre", left)
        blocks.append(Block(f"L{tag}_a_{u}", a + b1 + b2))
        return blocks
    # DMAs issued two steps ago (and earlier) have landed in every wave; the
    # 8 of the previous step may still be in flight, and so may the operand
    # reads that step issued last (from slots no DMA of this step writes).
    blocks.append(Block(f"L{tag}_s_{u}", [waitcnt(vm=8, lgkm=N_PRE_K + N_PRE_V), Ins("s_barrier", "barrier")]))
    if opt:
        if kind == "last":
            blocks += opt_tail(f"{tag}L", q, "last", False)
            blocks.append(Block(f"L{tag}_j_{u}", [branch("s_branch", end_label, cond=False)]))
            return blocks
        blocks.append(Block(f"L{tag}_mt_{u}", [salu(f"s_sub_u32 {sreg(S_T1)}, {sreg(S_R1)}, {s_in('it0')}"),
                                               salu(f"s_cmp_ge_u32 {sreg(S_T1)}, {sreg(S_SPAN)}"),
                                               branch("s_cbranch_scc1", f"L{tag}_am_{u}")]))
        for masked in (False, True):
            mt = "m" if masked else "u"
            bl = opt_tail(f"{tag}{mt}", q, kind, masked)
            bl[0].name = f"L{tag}_a{mt}_{u}"
            blocks += bl
            if not masked:
                blocks.append(Block(f"L{tag}_j_{u}", [branch("s_branch", end_label, cond=False)]))
        return blocks
    assert kind == "full"
    blocks += call_rescale(f"{tag}r0", par, 0)
    if kind == "last":
        a, left = block_a(q, "last", False)
        b1, left = block_b1(q, "last", False, left)
        blocks.append(Block(f"L{tag}_a_{u}", a + b1))
        blocks += call_rescale(f"{tag}r1", par, 1)
        blocks.append(Block(f"L{tag}_b2_{u}", block_b2(q, "last", left)))
        blocks.append(Block(f"L{tag}_j_{u}", [branch("s_branch", end_label, cond=False)]))
        return blocks
    # tile r + 1 needs the range mask iff it lies outside [it0, it1)
    blocks.append(Block(f"L{tag}_mt_{u}", [salu(f"s_sub_u32 {sreg(S_T1)}, {sreg(S_R1)}, {s_in('it0')}"),
                                           salu(f"s_cmp_ge_u32 {sreg(S_T1)}, {sreg(S_SPAN)}"),
                                           branch("s_cbranch_scc1", f"L{tag}_am_{u}")]))
    for masked in (False, True):
        mt = "m" if masked else "u"
        a, left = block_a(q, kind, masked)
        b1, left = block_b1(q, kind, masked, left)
        blocks.append(Block(f"L{tag}_a{mt}_{u}", a + b1))
        blocks += call_rescale(f"{tag}{mt}r1", par, 1)
        blocks.append(Block(f"L{tag}_b2{mt}_{u}", block_b2(q, kind, left)))
        if not masked:
            blocks.append(Block(f"L{tag}_j_{u}", [branch("s_branch", end_label, cond=False)]))
    return blocks


def prologue():
    """Q rows into their AGPRs, O = 0, constants, LDS operand addresses, the
    first three K tiles and the first two V^T tiles staged, then wait and
    barrier."""
    # Every lane runs the loop; the compiler's code before this block wrote
    # some of the input SGPRs with VALU instructions (v_readfirstlane), and a
    # buffer instruction reading such an SGPR needs 5 wait states, which the
    # compiler cannot see inside inline assembly.
    out = [salu("s_mov_b64 exec, -1"), Ins("s_nop 7", "nop")]
    for rb in range(2):
        for kk in range(8):
            d = Q_A + 8 * kk + 4 * rb
            out.append(Ins(f"buffer_load_dwordx4 {areg(d, 4)}, {s_in(f'qoff{rb}')}, {s_in('qrsrc')}, 0 offen offset:{32 * kk}",
                           "vmem_ld", set(), regs("a", d, 4), vm=True))
    out += [
        salu(f"s_mov_b32 {sreg(S_N)}, {s_in('ntiles')}"),
        salu(f"s_mov_b64 {sreg(S_KRS, 2)}, {s_in('kbase')}"),
        salu(f"s_mov_b32 {sreg(S_KBYTES)}, {s_in('kbytes')}"),
        salu(f"s_max_i32 {sreg(S_KRS + 2)}, {sreg(S_KBYTES)}, 0"),
        salu(f"s_mov_b32 {sreg(S_KRS + 3)}, {RSRC_WORD3:#x}"),
        salu(f"s_mov_b64 {sreg(S_VRS, 2)}, {s_in('vbase')}"),
        salu(f"s_lshl_b32 {sreg(S_VBYTES)}, {sreg(S_N)}, 14"),
        salu(f"s_max_i32 {sreg(S_VRS + 2)}, {sreg(S_VBYTES)}, 0"),
        salu(f"s_mov_b32 {sreg(S_VRS + 3)}, {RSRC_WORD3:#x}"),
        salu(f"s_mov_b32 {sreg(S_EIGHT)}, {EIGHT_BITS:#x}"),
        salu(f"s_mov_b32 {sreg(S_SENT)}, {SENTINEL_BITS:#x}"),
        salu(f"s_sub_i32 {sreg(S_SPAN)}, {s_in('it1')}, {s_in('it0')}"),
        salu(f"s_max_i32 {sreg(S_SPAN)}, {sreg(S_SPAN)}, 0"),
        salu(f"s_mov_b32 {sreg(S_R1)}, 0"),
        salu(f"s_mov_b32 {sreg(S_KEY0)}, {s_in('key0')}"),
    ]
    for f in range(4):
        out.append(salu(f"s_mov_b64 {sreg(S_FLAG + 2 * f, 2)}, 0"))
    # K(0), K(1), V^T(0), K(2), V^T(1) into their slots, in the order the
    # first steps need them: the pre step waits only for Q and K(0)
    for kind, slot in (("k", 0), ("k", 1), ("v", 0), ("k", 2), ("v", 1)):
        for i in range(4):
            out += dma(kind, i, slot)
        out += desc_advance(kind)
    # O = 0 by eight MFMAs of zero operands (instead of 128 AGPR writes)
    z = PK_V
    out += [valu(f"v_mov_b32 {vreg(z + k)}, 0", set(), {f"v{z + k}"}) for k in range(4)]
    for blk in range(8):
        out.append(mfma(("a", O_A + 16 * blk), ("v", z), ("v", z), False))
    for kk in range(8):
        out.append(valu(f"v_xor_b32 {vreg(KOFF_V + kk)}, {32 * kk}, {s_in('kofs')}", set(), {f"v{KOFF_V + kk}"}))
    for s2 in range(4):
        out.append(valu(f"v_xor_b32 {vreg(VOFF_V + s2)}, {32 * s2}, {s_in('vofs')}", set(), {f"v{VOFF_V + s2}"}))
        out.append(valu(f"v_add_u32 {vreg(VOFF_V + s2)}, {V_RING}, {vreg(VOFF_V + s2)}",
                        {f"v{VOFF_V + s2}"}, {f"v{VOFF_V + s2}"}))
    for rb in range(2):
        out += [
            valu(f"v_mov_b32 {vreg(V_KSR + rb)}, {s_in(f'ksr{rb}')}", set(), {f"v{V_KSR + rb}"}),
            valu(f"v_sub_u32 {vreg(V_SPAN + rb)}, {s_in(f'ker{rb}')}, {s_in(f'ksr{rb}')}", set(),
                 {f"v{V_SPAN + rb}"}),
            valu(f"v_max_i32 {vreg(V_SPAN + rb)}, 0, {vreg(V_SPAN + rb)}", {f"v{V_SPAN + rb}"},
                 {f"v{V_SPAN + rb}"}),
            valu(f"v_mov_b32 {vreg(V_L + rb)}, 0", set(), {f"v{V_L + rb}"}),
        ]
    for k in range(4):
        out.append(valu(f"v_mov_b32 {vreg(V_AL + k)}, 0", set(), {f"v{V_AL + k}"}))
    # n = -m c with m at the sentinel (no key seen yet)
    out += [valu(f"v_mov_b32 {vreg(V_NSENT)}, {sreg(S_SENT)}", {f"s{S_SENT}"}, {f"v{V_NSENT}"}),
            valu(f"v_mul_f32 {vreg(V_NSENT)}, {s_in('negc')}, {vreg(V_NSENT)}", {f"v{V_NSENT}"},
                 {f"v{V_NSENT}"}),
            valu(f"v_mov_b32 {vreg(V_NMCC)}, {vreg(V_NSENT)}", {f"v{V_NSENT}"}, {f"v{V_NMCC}"})]
    for k in range(4):
        out.append(valu(f"v_mov_b32 {vreg(V_NMC + k)}, {vreg(V_NSENT)}", {f"v{V_NSENT}"}, {f"v{V_NMC + k}"}))
    out.append(valu(f"v_mov_b32 {vreg(V_NINF)}, {NEG_INF_BITS:#x}", set(), {f"v{V_NINF}"}))
    out.append(valu(f"v_mov_b32 {vreg(V_THR)}, {THR_BITS:#x}", set(), {f"v{V_THR}"}))
    for f in (S_FORCE, S_FORCE1):
        out.append(salu(f"s_mov_b64 {sreg(f, 2)}, 0", set(), {f"s{f}", f"s{f + 1}"}))
    # Q and K(0) have landed in every wave (K(1), V^T(0), K(2), V^T(1) may
    # still be in flight: 16 DMAs)
    out += [waitcnt(vm=PRO_LATE), Ins("s_barrier", "barrier")]
    return out


def epilogue():
    """LSE = log2(l) + m c per row; O = acc / l as bf16 rows, staged through
    this wave's LDS region (32 rows at a 272-byte stride, then their 32 byte
    offsets) so that each store writes whole 256-byte rows."""
    out = [waitcnt(vm=0, lgkm=0), Ins("s_barrier", "barrier")]
    E = V_EPI
    lane = s_in("lane")
    # E+0: write base (row rl, hh half) ; E+1: offset-table slot of row rl
    # E+2: read base (row lane>>4, chunk lane&15) ; E+3: offset-table read base
    # E+4: 16 * (lane & 15) ; E+5, E+6: temporaries
    t5, t6 = E + 5, E + 6
    out += [
        valu(f"v_and_b32 {vreg(t5)}, 31, {lane}", set(), {f"v{t5}"}),
        valu(f"v_lshrrev_b32 {vreg(t6)}, 5, {lane}", set(), {f"v{t6}"}),
        valu(f"v_mul_u32_u24 {vreg(E)}, 0x110, {vreg(t5)}", {f"v{t5}"}, {f"v{E}"}),
        valu(f"v_lshl_add_u32 {vreg(E)}, {vreg(t6)}, 3, {vreg(E)}", {f"v{t6}", f"v{E}"}, {f"v{E}"}),
        valu(f"v_add_u32 {vreg(E)}, {s_in('ebase')}, {vreg(E)}", {f"v{E}"}, {f"v{E}"}),
        valu(f"v_lshl_add_u32 {vreg(E + 1)}, {vreg(t5)}, 2, {s_in('ebase')}", {f"v{t5}"}, {f"v{E + 1}"}),
        valu(f"v_add_u32 {vreg(E + 1)}, {32 * 272}, {vreg(E + 1)}", {f"v{E + 1}"}, {f"v{E + 1}"}),
        valu(f"v_lshrrev_b32 {vreg(t6)}, 4, {lane}", set(), {f"v{t6}"}),
        valu(f"v_and_b32 {vreg(E + 4)}, 15, {lane}", set(), {f"v{E + 4}"}),
        valu(f"v_lshlrev_b32 {vreg(E + 4)}, 4, {vreg(E + 4)}", {f"v{E + 4}"}, {f"v{E + 4}"}),
        valu(f"v_mul_u32_u24 {vreg(E + 2)}, 0x110, {vreg(t6)}", {f"v{t6}"}, {f"v{E + 2}"}),
        valu(f"v_add3_u32 {vreg(E + 2)}, {s_in('ebase')}, {vreg(E + 2)}, {vreg(E + 4)}",
             {f"v{E + 2}", f"v{E + 4}"}, {f"v{E + 2}"}),
        valu(f"v_lshl_add_u32 {vreg(E + 3)}, {vreg(t6)}, 2, {s_in('ebase')}", {f"v{t6}"}, {f"v{E + 3}"}),
        valu(f"v_add_u32 {vreg(E + 3)}, {32 * 272}, {vreg(E + 3)}", {f"v{E + 3}"}, {f"v{E + 3}"}),
    ]
    il = (V_T + 8, V_T + 9)
    for rb in range(2):
        out += swap_combine(V_L + rb, V_T + 2 + rb, "v_add_f32")
    for rb in range(2):
        t = V_T + rb
        nmc = V_NMC + 2 + rb      # -m c after the last half
        out += [
            valu(f"v_log_f32 {vreg(t)}, {vreg(V_L + rb)}", {f"v{V_L + rb}"}, {f"v{t}"}, trans=True),
            valu(f"v_sub_f32 {vreg(t)}, {vreg(t)}, {vreg(nmc)}", {f"v{nmc}", f"v{t}"}, {f"v{t}"}),
            Ins(f"buffer_store_dword {vreg(t)}, {s_in(f'lsoff{rb}')}, {s_in('lrsrc')}, 0 offen", "vmem_st",
                {f"v{t}"}, set(), vm=True),
            valu(f"v_rcp_f32 {vreg(il[rb])}, {vreg(V_L + rb)}", {f"v{V_L + rb}"}, {f"v{il[rb]}"}, trans=True),
        ]
    for rb in range(2):
        if rb == 1:
            out.append(waitcnt(lgkm=0))
        for db in range(4):
            for j in range(4):
                a0 = O_A + 32 * db + 16 * rb + 4 * j
                tv = 8 * (4 * db + j) % 64   # rotate through v[0:63]
                for k in range(4):
                    out.append(valu(f"v_accvgpr_read_b32 {vreg(tv + k)}, {areg(a0 + k)}", {f"a{a0 + k}"},
                                    {f"v{tv + k}"}))
                for k in range(4):
                    out.append(valu(f"v_mul_f32 {vreg(tv + k)}, {vreg(tv + k)}, {vreg(il[rb])}",
                                    {f"v{tv + k}", f"v{il[rb]}"}, {f"v{tv + k}"}))
                out.append(valu(f"v_cvt_pk_bf16_f32 {vreg(tv + 4)}, {vreg(tv)}, {vreg(tv + 1)}",
                                {f"v{tv}", f"v{tv + 1}"}, {f"v{tv + 4}"}))
                out.append(valu(f"v_cvt_pk_bf16_f32 {vreg(tv + 5)}, {vreg(tv + 2)}, {vreg(tv + 3)}",
                                {f"v{tv + 2}", f"v{tv + 3}"}, {f"v{tv + 5}"}))
                out.append(Ins(f"ds_write_b64 {vreg(E)}, {vreg(tv + 4, 2)} offset:{64 * db + 16 * j}", "lds_w",
                               {f"v{E}", f"v{tv + 4}", f"v{tv + 5}"}, set(), lgkm=True))
        out.append(Ins(f"ds_write_b32 {vreg(E + 1)}, {s_in(f'ooff{rb}')}", "lds_w", {f"v{E + 1}"}, set(),
                       lgkm=True))
        out.append(waitcnt(lgkm=0))
        for i in range(8):
            out.append(Ins(f"ds_read_b32 {vreg(64 + i)}, {vreg(E + 3)} offset:{16 * i}", "lds",
                           {f"v{E + 3}"}, {f"v{64 + i}"}, lgkm=True))
            out.append(Ins(f"ds_read_b128 {vreg(72 + 4 * i, 4)}, {vreg(E + 2)} offset:{4 * 272 * i}", "lds",
                           {f"v{E + 2}"}, regs("v", 72 + 4 * i, 4), lgkm=True))
        for i in range(8):
            out.append(valu(f"v_add_u32 {vreg(64 + i)}, {vreg(64 + i)}, {vreg(E + 4)}",
                            {f"v{64 + i}", f"v{E + 4}"}, {f"v{64 + i}"}))
            out.append(Ins(f"buffer_store_dwordx4 {vreg(72 + 4 * i, 4)}, {vreg(64 + i)}, {s_in('orsrc')}, 0 offen",
                           "vmem_st", regs("v", 72 + 4 * i, 4) | {f"v{64 + i}"}, set(), vm=True))
    return out


def program():
    u = "%="
    blocks = [Block(f"Lpro_{u}", prologue() + [salu(f"s_cmp_le_i32 {sreg(S_N)}, 0"),
                                                  branch("s_cbranch_scc1", f"Lepi_{u}")])]
    blocks += step_blocks("p", 3, "pre", None)
    blocks.append(Block(f"Lr0_{u}", [salu(f"s_mov_b32 {sreg(S_R1)}, 1")]))
    # Step 0 takes the exact running max of tile 1 (as the pre step does of
    # tile 0), so that every row whose range starts within the first two
    # tiles has a finite max before the steps without one; it is phase 0.
    blocks.append(Block(f"Le_{u}", [salu(f"s_cmp_ge_i32 {sreg(S_R1)}, {sreg(S_N)}"),
                                    branch("s_cbranch_scc1", f"Llast0_{u}")]))
    blocks += step_blocks("e", 0, "full", f"Leinc_{u}", opt=False)
    blocks.append(Block(f"Leinc_{u}", [salu(f"s_add_u32 {sreg(S_R1)}, {sreg(S_R1)}, 1")]))
    # the loop, laid out from phase 1 (step 0 falls into it there)
    for q in (1, 2, 3, 0):
        blocks.append(Block(f"Lt{q}_{u}", [salu(f"s_cmp_ge_i32 {sreg(S_R1)}, {sreg(S_N)}"),
                                          branch("s_cbranch_scc1", f"Llast{q}_{u}")]))
        blocks += step_blocks(f"f{q}", q, "full", f"Linc{q}_{u}")
        tail = [salu(f"s_add_u32 {sreg(S_R1)}, {sreg(S_R1)}, 1")]
        if q == 0:
            tail.append(branch("s_branch", f"Lt1_{u}", cond=False))
        blocks.append(Block(f"Linc{q}_{u}", tail))
    for q in range(4):
        bl = step_blocks(f"l{q}", q, "last", f"Lepi_{u}")
        bl[0].name = f"Llast{q}_{u}"
        blocks += bl
    # the out-of-line calls, then the shared rescale and recompute routines
    # (reached only by branches)
    blocks += COLD
    COLD.clear()
    blocks.append(Block(f"Lrescale_{u}", rescale_routine()))
    for par in range(2):
        for h in range(2):
            blocks.append(Block(f"Lrecomp{par}{h}_{u}", recompute_routine(par, h)))
    blocks.append(Block(f"Lepi_{u}", epilogue()))
    return blocks


# ---------------------------------------------------------------------------
# hazard padding over the control-flow graph, and wait counts
# ---------------------------------------------------------------------------

SAT = 64
MFMA_RAW = 12       # XDL 8-pass result -> any non-MFMA read, or a non-MFMA overwrite
VALU_TO_MFMA = 2    # VALU write -> MFMA operand read
VALU_SGPR_MASK = 2  # VALU write of an SGPR pair -> VALU read of it as lane mask / carry
VALU_TO_PERM = 2    # VALU write -> v_permlane32_swap read
TRANS_FWD = 1       # transcendental result -> next VALU read
M0_TO_DMA = 1       # SALU write of M0 -> LDS DMA
AB_WAR = 4          # margin: MFMA srcA/B read -> overwrite


class HState:
    def __init__(self):
        self.mf_w = {}      # reg -> (dist, dst key)
        self.mf_ab = {}     # reg -> dist since an MFMA read it as srcA/B
        self.valu_w = {}    # reg -> dist since a VALU wrote it
        self.trans_w = {}
        self.m0 = SAT

    def copy(self):
        h = HState()
        h.mf_w = dict(self.mf_w)
        h.mf_ab = dict(self.mf_ab)
        h.valu_w = dict(self.valu_w)
        h.trans_w = dict(self.trans_w)
        h.m0 = self.m0
        return h

    def advance(self, n):
        for d in (self.valu_w, self.trans_w, self.mf_ab):
            for k in list(d):
                v = d[k] + n
                if v >= SAT:
                    del d[k]
                else:
                    d[k] = v
        for k in list(self.mf_w):
            v, key = self.mf_w[k]
            v += n
            if v >= SAT:
                del self.mf_w[k]
            else:
                self.mf_w[k] = (v, key)
        self.m0 = min(SAT, self.m0 + n)

    def merge(self, o):
        h = self.copy()
        for k, v in o.valu_w.items():
            h.valu_w[k] = min(v, h.valu_w.get(k, SAT))
        for k, v in o.trans_w.items():
            h.trans_w[k] = min(v, h.trans_w.get(k, SAT))
        for k, v in o.mf_ab.items():
            h.mf_ab[k] = min(v, h.mf_ab.get(k, SAT))
        for k, (v, key) in o.mf_w.items():
            if k in h.mf_w:
                v0, key0 = h.mf_w[k]
                h.mf_w[k] = (min(v, v0), key if key == key0 else None)
            else:
                h.mf_w[k] = (v, key)
        h.m0 = min(h.m0, o.m0)
        return h

    def key(self):
        return (tuple(sorted(self.mf_w.items())), tuple(sorted(self.mf_ab.items())),
                tuple(sorted(self.valu_w.items())), tuple(sorted(self.trans_w.items())), self.m0)


def need(ins, h):
    """Wait states that must separate ins from what came before."""
    n = 0
    if ins.kind == "mfma":
        dkey, ab, csrc = ins.mfma
        for r in ab:
            if r in h.mf_w:
                n = max(n, MFMA_RAW - h.mf_w[r][0])
            if r in h.valu_w:
                n = max(n, VALU_TO_MFMA - h.valu_w[r])
        if csrc:
            for r in csrc:
                if r in h.mf_w:
                    d, key = h.mf_w[r]
                    if key != dkey:
                        n = max(n, MFMA_RAW - d)
                if r in h.valu_w:
                    n = max(n, VALU_TO_MFMA - h.valu_w[r])
        for r in ins.wr:
            if r in h.valu_w:
                n = max(n, VALU_TO_MFMA - h.valu_w[r])
            if not csrc and r in h.mf_w:
                n = max(n, MFMA_RAW - h.mf_w[r][0])
        return n
    for r in ins.rd | ins.mask_rd:
        if r in h.mf_w:
            n = max(n, MFMA_RAW - h.mf_w[r][0])
    for r in ins.wr:
        if r in h.mf_w:
            n = max(n, MFMA_RAW - h.mf_w[r][0])
        if r in h.mf_ab:
            n = max(n, AB_WAR - h.mf_ab[r])
    if ins.kind in ("valu", "perm"):
        for r in ins.mask_rd | {x for x in ins.rd if x.startswith("s")}:
            if r in h.valu_w:
                n = max(n, VALU_SGPR_MASK - h.valu_w[r])
        if ins.kind == "perm":
            for r in ins.rd:
                if r in h.valu_w:
                    n = max(n, VALU_TO_PERM - h.valu_w[r])
        if not ins.trans:
            for r in ins.rd:
                if r in h.trans_w:
                    n = max(n, TRANS_FWD - h.trans_w[r])
    if ins.kind == "dma":
        n = max(n, M0_TO_DMA - h.m0)
    return max(n, 0)


def apply(ins, h):
    if ins.kind == "label":
        return
    if ins.kind == "nop":
        h.advance(int(ins.text.split()[1]) + 1)
        return
    h.advance(1)
    if ins.kind == "mfma":
        dkey, ab, csrc = ins.mfma
        for r in ins.wr:
            h.mf_w[r] = (0, dkey)
            h.valu_w.pop(r, None)
        for r in ab:
            h.mf_ab[r] = 0
        return
    for r in ins.wr:
        if r == "m0":
            h.m0 = 0
        h.mf_w.pop(r, None)
        if ins.kind in ("valu", "perm"):
            h.valu_w[r] = 0
            if ins.trans:
                h.trans_w[r] = 0
            else:
                h.trans_w.pop(r, None)
        else:
            h.valu_w.pop(r, None)
            h.trans_w.pop(r, None)


def pad_block(ins_list, h):
    out = []
    for ins in ins_list:
        n = need(ins, h)
        while n > 0:
            k = min(n, 16)
            nop = Ins(f"s_nop {k - 1}", "nop")
            out.append(nop)
            apply(nop, h)
            n -= k
        out.append(ins)
        apply(ins, h)
    return out


def successors(blocks):
    names = {b.name: i for i, b in enumerate(blocks)}
    succ = []
    for i, b in enumerate(blocks):
        s = []
        last = b.ins[-1] if b.ins else None
        if last is not None and last.kind in ("branch", "call"):
            s.append(names[last.branch])
            if last.cond and i + 1 < len(blocks):
                s.append(i + 1)
        elif last is not None and last.kind == "ret":
            s += [k for k, x in enumerate(blocks) if x.ret_point]
        elif i + 1 < len(blocks):
            s.append(i + 1)
        succ.append(s)
    return succ


def pad_program(blocks):
    succ = successors(blocks)
    preds = [[] for _ in blocks]
    for i, s in enumerate(succ):
        for j in s:
            preds[j].append(i)
    entry = [None] * len(blocks)
    entry[0] = HState()
    exit_ = [None] * len(blocks)
    padded = [None] * len(blocks)
    work = list(range(len(blocks)))
    while work:
        i = work.pop(0)
        h = None
        for p in preds[i]:
            if exit_[p] is not None:
                h = exit_[p] if h is None else h.merge(exit_[p])
        if i == 0:
            h = HState()
        if h is None:
            continue
        if entry[i] is not None and entry[i].key() == h.key() and padded[i] is not None:
            continue
        entry[i] = h
        hh = h.copy()
        padded[i] = pad_block(blocks[i].ins, hh)
        exit_[i] = hh
        for j in succ[i]:
            if j not in work:
                work.append(j)
    for i, b in enumerate(blocks):
        assert padded[i] is not None, f"unreachable block {b.name}"
    return padded


PAIR_AGE = 3         # MFMAs since a read was issued before it is taken as landed


def insert_waits(blocks):
    """s_waitcnt lgkmcnt(n) before each use of an LDS read's result, with n
    the number of LDS operations issued after that read.  The queue of
    outstanding LDS operations is carried along the control-flow graph; every
    block's predecessors must agree on it (checked).  Results of memory loads
    (the Q rows) are only used after a vmcnt(0); the DMAs write no
    registers and are waited for explicitly at each step."""
    succ = successors(blocks)
    entry = [None] * len(blocks)
    entry[0] = ([], ())
    out = []
    for i, b in enumerate(blocks):
        assert entry[i] is not None, f"block {b.name} has no forward predecessor"
        lg = [set(x) for x in entry[i][0]]
        born = [-PAIR_AGE] * len(lg)        # MFMA count when each read was issued
        n_mf = 0
        vmq = list(entry[i][1])             # outstanding memory operations (registers they load)
        res = []
        for ins in b.ins:
            if ins.kind == "wait":
                mm = re.search(r"lgkmcnt\((\d+)\)", ins.text)
                if mm:
                    k = int(mm.group(1))
                    if k < len(lg):
                        lg, born = (lg[len(lg) - k:], born[len(born) - k:]) if k else ([], [])
                mv = re.search(r"vmcnt\((\d+)\)", ins.text)
                if mv:
                    k = int(mv.group(1))
                    vmq = vmq[len(vmq) - k:] if 0 < k < len(vmq) else ([] if k == 0 else vmq)
                res.append(ins)
                continue
            uses = ins.rd | ins.mask_rd | ins.wr
            pend_vm = set().union(*vmq) if vmq else set()
            assert not (uses & pend_vm), f"memory load result used before its vmcnt wait: {ins.text}"
            w_l = None
            for k, regset in enumerate(lg):
                if regset & uses:
                    w_l = len(lg) - k - 1
            if w_l is not None:
                # an MFMA also waits for the next read when that one is old
                # enough to have landed: the next MFMA then needs no wait
                if ins.kind == "mfma" and w_l >= 1 and n_mf - born[len(lg) - w_l] >= PAIR_AGE:
                    w_l -= 1
                res.append(waitcnt(lgkm=w_l))
                lg, born = (lg[len(lg) - w_l:], born[len(born) - w_l:]) if w_l > 0 else ([], [])
            if ins.lgkm and len(lg) >= 15:      # the lgkmcnt field holds at most 15
                res.append(waitcnt(lgkm=7))
                lg, born = lg[len(lg) - 7:], born[len(born) - 7:]
            res.append(ins)
            if ins.kind == "mfma":
                n_mf += 1
            if ins.lgkm:
                lg.append(set(ins.wr))
                born.append(n_mf)
            if ins.vm:
                vmq.append(frozenset(ins.wr) if ins.kind == "vmem_ld" else frozenset())
        out.append(res)
        # outstanding memory operations matter only while a load among them
        # still has registers to wait for
        state = ([set(x) for x in lg], tuple(vmq) if any(vmq) else ())
        for j in succ[i]:
            if entry[j] is None:
                entry[j] = state
                continue
            m = _merge_queues(entry[j], state)
            assert m is not None, f"LDS queues differ into {blocks[j].name}"
            assert j > i or m == entry[j], f"back edge with a longer LDS queue into {blocks[j].name}"
            entry[j] = m
    return out


def _merge_queues(a, b):
    """Entry state of a block reached with LDS queues a and b: the longer
    one, when the shorter is its tail (a wait counted against the longer
    queue is then also enough for the shorter); None otherwise."""
    if a[1] != b[1]:
        return None
    la, lb = a[0], b[0]
    if len(la) < len(lb):
        la, lb = lb, la
        a, b = b, a
    if lb and la[len(la) - len(lb):] != lb:
        return None
    return a


def generate():
    blocks = program()
    check_returns(blocks)
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
    c = [f"v{i}" for i in range(V_LIMIT)] + [f"a{i}" for i in range(256)]
    c += [f"s{i}" for i in range(S_FIRST, S_LASTC + 1)]
    c += ["vcc", "exec", "m0", "memory"]
    return c


def emit(path):
    lines = generate()
    with open(path, "w") as f:
        f.write("// Generated by gen_fwd_wide.py: the tile loop of fwd_wide_kernel.  Do not edit.\n")
        f.write("#pragma once\n")
        f.write("#define SWATTN_FWD_WIDE_ASM \\\n")
        for ln in lines:
            f.write(f'  "{ln}\\n" \\\n')
        f.write('  ""\n')
        f.write(f"#define SWATTN_FWD_WIDE_LDS_BYTES {LDS_BYTES}\n")
        f.write("#define SWATTN_FWD_WIDE_CLOBBERS \\\n  ")
        f.write(", ".join(f'"{x}"' for x in clobbers()))
        f.write("\n")
    return len(lines)


if __name__ == "__main__":
    n = emit(sys.argv[1])
    print(f"{n} lines")
