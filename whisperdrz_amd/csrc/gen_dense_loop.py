"""Generates dense_loop.inc: the hand-scheduled main loop of dense_pipe_kernel (attn_dense.hip).

Usage: python gen_dense_loop.py [out_path]   (whisperdrz_amd/build.py runs it before compiling)

The loop is one inline-asm statement per element type (bf16 / fp16) and form over physical
registers that the kernel binds with register constraints. Design (one wavefront per SIMD, 96
queries per wavefront as three 32-query blocks b = 0, 1, 2 -- or, in the two-block form, 64 as
blocks 0, 1 with two phases per step, block 1 in the role of block 2 below; 32 keys per step,
64-key LDS tiles):

  * Each step s runs three phases. Phase b runs the online softmax of block b's scores S(s)[b]
    on the VALU (exp2, bf16/fp16 packs of P, row sums, the rescale check) while the matrix pipe
    runs the MFMAs of the previous block: in phase 1 and 2 those of blocks 0 and 1 (P(s)V(s) and
    the next step's scores S(s+1) = K(s+1) Q^T), in phase 0 those of block 2 of the previous step
    (P(s-1)V(s-1) and S(s)[2]). Every MFMA input was produced at least one phase earlier and every
    VALU input at least one phase earlier, so no instruction waits on the one just issued: the
    in-order instruction stream keeps the matrix pipe and the VALU busy side by side (8 MFMAs and
    ~45 VALU instructions per phase, ~5 VALU instructions between MFMAs).
  * The running max is subtracted inside the MFMA: every score chain starts from cinit[b] =
    -m_run[b]. The rescale check runs on the step's row sum (a lane's 16 P values summing above
    1024 means a score exceeded the max by more than 6 in log2 units); the rare rescale takes
    the true max, rescales O (AGPRs), l and cinit, and redoes the block's softmax. The running
    max starts at the true max of the first step: the prologue computes every block's step-0
    scores and takes their row max before the loop. The compare is
    placed a few instructions before the phase's branch (a branch on a VCC the VALU has only just
    written stalls the in-order wavefront).
  * K and V operands for the MFMAs come from LDS one step ahead into double-buffered AGPRs
    (K through ds_read_b128 in the permuted key order that makes P^T the B operand without
    shuffles; V^T through ds_read_b64_tr_b16). Tiles of 64 keys go global -> LDS directly (buffer
    loads to LDS, 1 KB = 8 rows per instruction) through four LDS buffers of unpadded 128-byte rows
    whose 16-byte chunks are XOR-swizzled by (row / 2) % 8 (a lane fetches the global chunk that
    the swizzle puts at its LDS position); tile t+3 is requested during tile t and tile t+2 must have
    landed by tile t's barrier (one workgroup barrier per tile). The loads are bounded by the
    tensor's extent (rows past the last key read as zero; those keys are never used unmasked).
  * The kernel is persistent; during the first 12 iterations of an item each wavefront also
    requests one 1 KB piece of the next item's Q rows straight into LDS (buffer loads to LDS).

Register map (the kernel passes these through "{v[..]}" / "{a[..]}" constraints):
  v0-47 S[b] (16 each)   v48-95 cinit[b]   v96-119 P[b] (8 each: two 16-key chunks)
  v120-135 exp temps     v136-139 K read lane bases   v140-147 V^T read lane bases   v148-151 K reads
  v152-154 m_run[b]      v156-158 l_run[b] (this lane's half of the row sum)   v159 -inf
  v163 8 * (lane >> 5)   v164-167 global byte offsets of this lane's tile rows (K r, r+8, V r, r+8)
  v168-171 V^T reads of tile t
  v172-183 rare-path temporaries   v184-207 row-sum temporaries (8 per block)
  v208-211 V^T reads of tile t+1   v212-215 the tail's   v224 Q prefetch lane offset   v225 its address
  a0-95 O[b][db] (16 each)   a96-143 Q[b][ks] (4 each)   a144-175 K buffers (2 x 16)
  a176-207 V buffers (2 x 16: [ch][db] operands of 4)
  s70-s79 loop state (clobbered: iteration, tile offsets, sum limit, rescale floor); the kernel
  passes the buffer resources of K, V and the next item's Q rows in s[80:83], s[84:87], s[88:91].
"""
import sys
from pathlib import Path

# ---- register map --------------------------------------------------------------------------
def S(b): return 16 * b
def CINIT(b): return 48 + 16 * b
def P(b, ch=0): return 96 + 8 * b + 4 * ch
T0 = 120
KL = 136   # 136..139 K read lane bases, one per 16-key chunk ks (the layout is XOR-swizzled)
VL = 140   # 140..147 V^T read lane bases [db][s]: dims 32 db.., rows +4 s
QVOFF, QV = 224, 225  # the Q prefetch: this lane's row offset, and the piece's address
def U(b): return 184 + 8 * b  # row-sum temporaries of block b (184..207)
def MRUN(b): return 152 + b
def LRUN(b): return 156 + b  # a 3-register tuple (even-aligned), an output of the loop
HL8 = 163  # 8 * (lane >> 5), the masking's key offset
VOFF = 164  # 164..167 global byte offsets of this lane's tile rows (K r, K r+8, V r, V r+8)
KADDR = 148   # 148..151 the K read addresses of an iteration (per ks)
VADDRA = 168  # 168..171 the V^T read addresses of tile t ([db][s])
VADDRB = 208  # 208..211 the same for tile t+1
VADDRT = 212  # 212..215 the same for the tail
RT = 172  # rare-path temporaries 172..183
NEGINF = 159  # -inf (the masked score)
def O(b, db): return 32 * b + 16 * db
def Q(b, ks): return 96 + 16 * b + 4 * ks
def KB(p, ks): return 144 + 16 * p + 4 * ks
def VB(p, ch, db): return 176 + 16 * p + 8 * ch + 4 * db

S_N = None  # the iteration count comes in through an operand: %[n]
S_IT, S_BUFA, S_BUFB, S_BUFC, S_TMP = "s70", "s71", "s72", "s73", "s74"
S_LIMIT = "s76"
SRD_K, SRD_V, SRD_Q = "s[80:83]", "s[84:87]", "s[88:91]"

TILE_BYTES = 64 * 128      # one 64-key tile of K (or V): 64 rows of 128 bytes, 16-byte chunks
HALF_BYTES = 32 * 128      # XOR-swizzled (chunk c of row r at byte 16 (c ^ ((r >> 1) & 7)))
ROW_BYTES = 128
V_BASE = 4 * TILE_BYTES    # the V tiles follow the four K tiles
SUM_LIMIT = "0x44800000"   # 1024.0f


def vr(lo, n=1):
    return f"v{lo}" if n == 1 else f"v[{lo}:{lo + n - 1}]"


def ar(lo, n=1):
    return f"a{lo}" if n == 1 else f"a[{lo}:{lo + n - 1}]"


class Gen:
    def __init__(self, dtype, nb=3):
        self.nb = nb  # 32-query blocks per wavefront (3: 96 queries, 2: 64)
        self.mfma = "v_mfma_f32_32x32x16_bf16" if dtype == "bf16" else "v_mfma_f32_32x32x16_f16"
        self.cvt = "v_cvt_pk_bf16_f32" if dtype == "bf16" else "v_cvt_pk_f16_f32"
        self.out = []
        self.rare = []

    def emit(self, s, into=None):
        (self.out if into is None else into).append(s)

    # ---- building blocks ---------------------------------------------------------------------
    def mfma_s(self, b, ks, kbuf):
        c = vr(CINIT(b), 16) if ks == 0 else vr(S(b), 16)
        return f"{self.mfma} {vr(S(b), 16)}, {ar(KB(kbuf, ks), 4)}, {ar(Q(b, ks), 4)}, {c}"

    def mfma_pv(self, b, ch, db, vbuf):
        return f"{self.mfma} {ar(O(b, db), 16)}, {ar(VB(vbuf, ch, db), 4)}, {vr(P(b, ch), 4)}, {ar(O(b, db), 16)}"

    def softmax_valu(self, b, check=True):
        """exp2 of the 16 scores, the row sum into T0 (pairs, then a tree), the rescale check into
        vcc, then the packs of P. The compare comes two MFMA slots before the phase's branch: a
        branch on a VCC that the VALU has only just written stalls the wavefront."""
        v = []
        for i in range(16):
            v.append(f"v_exp_f32 {vr(T0 + i)}, {vr(S(b) + i)}")
        for j in range(8):
            v.append(f"v_add_f32 {vr(U(b) + j)}, {vr(T0 + 2 * j)}, {vr(T0 + 2 * j + 1)}")
        for k in range(4):
            v.append(f"v_add_f32 {vr(U(b) + 2 * k)}, {vr(U(b) + 2 * k)}, {vr(U(b) + 2 * k + 1)}")
        v.append(f"v_add_f32 {vr(U(b))}, {vr(U(b))}, {vr(U(b) + 2)}")
        v.append(f"v_add_f32 {vr(U(b) + 4)}, {vr(U(b) + 4)}, {vr(U(b) + 6)}")
        v.append(f"v_add_f32 {vr(U(b))}, {vr(U(b))}, {vr(U(b) + 4)}")
        if check:
            # sum > limit in any lane -> rescale
            v.append(f"v_cmp_lt_f32 vcc, {S_LIMIT}, {vr(U(b))}")
        for j in range(8):
            v.append(f"{self.cvt} {vr(P(b) + j)}, {vr(T0 + 2 * j)}, {vr(T0 + 2 * j + 1)}")
        return v

    def row_max(self, b, mx):
        """mx = the max of block b's scores over the row (this lane's 16 and its partner lane's
        l ^ 32); uses mx + 1."""
        s0 = S(b)
        v = [f"v_max3_f32 {vr(mx)}, {vr(s0)}, {vr(s0 + 1)}, {vr(s0 + 2)}"]
        for i in range(3, 15, 2):
            v.append(f"v_max3_f32 {vr(mx)}, {vr(mx)}, {vr(s0 + i)}, {vr(s0 + i + 1)}")
        v.append(f"v_max_f32 {vr(mx)}, {vr(mx)}, {vr(s0 + 15)}")
        v.append(f"v_mov_b32 {vr(mx + 1)}, {vr(mx)}")
        v.append("s_nop 1")
        v.append(f"v_permlane32_swap_b32 {vr(mx)}, {vr(mx + 1)}")
        v.append(f"v_max_f32 {vr(mx)}, {vr(mx)}, {vr(mx + 1)}")
        return v

    def rare_block(self, b, label, back):
        """Rescale of block b (rare): the step's true max, O / l / cinit rescaled, softmax redone."""
        r = self.rare
        r.append(f"{label}:")
        r.append("s_nop 7")
        r.append("s_nop 7")
        mx, dl, al = RT, RT + 2, RT + 3
        r.extend(self.row_max(b, mx))
        r.append(f"v_max_f32 {vr(dl)}, 0, {vr(mx)}")  # delta >= 0: the max only grows
        r.append(f"v_add_f32 {vr(MRUN(b))}, {vr(MRUN(b))}, {vr(dl)}")
        r.append(f"v_exp_f32_e64 {vr(al)}, -{vr(dl)}")
        r.append("s_nop 1")  # a transcendental's result is not forwarded to the next VALU instruction
        r.append(f"v_mul_f32 {vr(LRUN(b))}, {vr(LRUN(b))}, {vr(al)}")
        tmp = [RT + 4 + i for i in range(8)]
        for i0 in range(0, 32, 8):
            for i in range(8):
                r.append(f"v_accvgpr_read_b32 {vr(tmp[i])}, {ar(O(b, 0) + i0 + i)}")
            for i in range(8):
                r.append(f"v_mul_f32 {vr(tmp[i])}, {vr(al)}, {vr(tmp[i])}")
            for i in range(8):
                r.append(f"v_accvgpr_write_b32 {ar(O(b, 0) + i0 + i)}, {vr(tmp[i])}")
        for i in range(16):
            r.append(f"v_sub_f32 {vr(CINIT(b) + i)}, 0, {vr(MRUN(b))}")
        for i in range(16):
            r.append(f"v_sub_f32 {vr(S(b) + i)}, {vr(S(b) + i)}, {vr(dl)}")
        r.extend(self.softmax_valu(b, check=False))
        r.append("s_nop 4")
        r.append(f"s_branch {back}")

    def mask_valu(self, b):
        """Keys past Lk (last step only): score -> -inf. Key of accumulator i of lane half hl:
        k0 + 8 hl + 16 (i >> 3) + (i & 7); valid iff 8 hl < rem - 16 (i >> 3) - (i & 7), rem = Lk - k0."""
        v = []
        for i in range(16):
            c = 16 * (i >> 3) + (i & 7)
            v.append(f"s_sub_i32 {S_TMP}, %[rem], {c}")
            v.append(f"v_cmp_gt_i32 vcc, {S_TMP}, {vr(HL8)}")
            v.append(f"v_cndmask_b32 {vr(S(b) + i)}, {vr(NEGINF)}, {vr(S(b) + i)}, vcc")
        return v

    def phase(self, p, ph, tag, pre=(), slots=None, do_s=True, mask=False):
        """One phase of a step of parity p: the softmax of block ph beside the MFMAs of the block
        before it (P V, and unless do_s is false the scores of its next step). slots: {MFMA
        index: [instructions after it]}. mask: the step is the last one and may hold keys past Lk."""
        slots = slots or {}
        if ph == 0:
            mb, kbuf, vbuf = self.nb - 1, p, 1 - p
        else:
            mb, kbuf, vbuf = ph - 1, 1 - p, p
        mf = []
        for ks in range(4):
            if do_s:
                mf.append(self.mfma_s(mb, ks, kbuf))
            ch, db = divmod(ks, 2)
            mf.append(self.mfma_pv(mb, ch, db, vbuf))
        valu = (self.mask_valu(ph) if mask else []) + self.softmax_valu(ph)
        for x in pre:
            self.emit(x)
        # spread the VALU list over the MFMA slots
        n, m = len(valu), len(mf)
        k = 0
        for i in range(m):
            self.emit(mf[i])
            for x in slots.get(i, []):
                self.emit(x)
            hi = (n * (i + 1)) // m
            while k < hi:
                self.emit(valu[k])
                k += 1
        # rescale when some lane's sum exceeded the limit (vcc, set by the compare above)
        label = f"R{tag}_%="
        back = f"B{tag}_%="
        self.emit(f"s_cbranch_vccnz {label}")
        self.emit(f"{back}:")
        self.emit(f"v_add_f32 {vr(LRUN(ph))}, {vr(LRUN(ph))}, {vr(U(ph))}")
        self.rare_block(ph, label, back)

    def final_pv(self, vbuf):
        """P V of the last block of the last step (the loop leaves it to the next step's phase 0)."""
        for ks in range(4):
            ch, db = divmod(ks, 2)
            self.emit(self.mfma_pv(self.nb - 1, ch, db, vbuf))

    def read_slots(self, kr, vrd):
        """The slots of a step's last phases that take the K reads (after the scores' MFMAs that
        use the other K buffer) and the V^T reads (once phase 0's P V is issued)."""
        if self.nb == 3:
            return {3: kr[:2], 4: kr[2:]}, {1: vrd[0:2], 2: vrd[2:4], 3: vrd[4:6], 4: vrd[6:8]}
        return {}, {1: vrd[0:2], 2: vrd[2:4], 3: kr[:2] + vrd[4:6], 4: kr[2:] + vrd[6:8]}

    def k_reads(self, p):
        """K(s+2) -> K buffer p: tile t+1, half p (base KADDR)."""
        return [f"ds_read_b128 {ar(KB(p, ks), 4)}, {vr(KADDR + ks)} offset:{p * HALF_BYTES}" for ks in range(4)]

    def v_reads(self, p, base=None):
        """V(s+1) -> V buffer 1-p: step 2t: tile t half 1 (VADDRA); step 2t+1: tile t+1 half 0 (VADDRB)."""
        b0, half = (VADDRA, 1) if p == 0 else (VADDRB, 0)
        base = b0 if base is None else base
        out = []
        for ch in range(2):
            for db in range(2):
                off = V_BASE + half * HALF_BYTES + ch * 16 * ROW_BYTES
                dst = VB(1 - p, ch, db)
                out.append(f"ds_read_b64_tr_b16 {ar(dst, 2)}, {vr(base + 2 * db)} offset:{off}")
                out.append(f"ds_read_b64_tr_b16 {ar(dst + 2, 2)}, {vr(base + 2 * db + 1)} offset:{off}")
        return out

    def tile_dma(self):
        """This wavefront's 16 rows of K and of V of one tile (four 1 KB pieces of 8 rows) straight
        into the LDS buffer at S_BUFC (LDS DMA at m0): lane l fetches the global chunk that the
        swizzle puts at position l % 8 of row l / 8 (the C++ side sets VOFF so)."""
        out = [f"s_add_u32 {S_TMP}, {S_BUFC}, %[dmab]"]
        for i, (srd, off) in enumerate(((SRD_K, 0), (SRD_K, 8 * ROW_BYTES), (SRD_V, V_BASE),
                                         (SRD_V, V_BASE + 8 * ROW_BYTES))):
            out.append(f"s_add_u32 m0, {S_TMP}, {off}" if off else f"s_mov_b32 m0, {S_TMP}")
            out.append("s_nop 0")
            out.append(f"buffer_load_dwordx4 {vr(VOFF + i)}, {srd}, 0 offen lds")
        return out

    def advance(self):
        return [
            f"v_add_u32 {vr(VOFF)}, %[tsk], {vr(VOFF)}",
            f"v_add_u32 {vr(VOFF + 1)}, %[tsk], {vr(VOFF + 1)}",
            f"v_add_u32 {vr(VOFF + 2)}, %[tsv], {vr(VOFF + 2)}",
            f"v_add_u32 {vr(VOFF + 3)}, %[tsv], {vr(VOFF + 3)}",
        ]

    def iteration(self, it):
        """One tile t: steps 2t and 2t+1, with tile t+3 requested (LDS DMA) into the buffer that
        tile t-1 held; tile t+2 (requested during tile t-1) must have landed by the barrier."""
        e = self.emit
        e(f"s_and_b32 {S_TMP}, {S_IT}, 3")
        e(f"s_mul_i32 {S_BUFA}, {S_TMP}, {TILE_BYTES}")
        e(f"s_add_u32 {S_TMP}, {S_IT}, 1")
        e(f"s_and_b32 {S_TMP}, {S_TMP}, 3")
        e(f"s_mul_i32 {S_BUFB}, {S_TMP}, {TILE_BYTES}")
        e(f"s_add_u32 {S_TMP}, {S_IT}, 3")
        e(f"s_and_b32 {S_TMP}, {S_TMP}, 3")
        e(f"s_mul_i32 {S_BUFC}, {S_TMP}, {TILE_BYTES}")
        for i in range(4):
            e(f"v_add_u32 {vr(KADDR + i)}, {S_BUFB}, {vr(KL + i)}")
        for i in range(4):
            e(f"v_add_u32 {vr(VADDRA + i)}, {S_BUFA}, {vr(VL + i)}")
        for i in range(4):
            e(f"v_add_u32 {vr(VADDRB + i)}, {S_BUFB}, {vr(VL + i)}")
        ld, adv = self.tile_dma(), self.advance()
        kr0, vr0 = self.k_reads(0), self.v_reads(0)
        kr1, vr1 = self.k_reads(1), self.v_reads(1)
        # step 2t (parity 0)
        last = self.nb - 1
        ks0, vs0 = self.read_slots(kr0, vr0)
        ks1, vs1 = self.read_slots(kr1, vr1)
        self.phase(0, 0, f"0P0{it}")
        if self.nb == 3:
            self.phase(0, 1, f"1P0{it}", pre=["s_waitcnt lgkmcnt(0)"], slots=ks0)
            self.phase(0, 2, f"2P0{it}", slots=vs0)
        else:
            self.phase(0, 1, f"1P0{it}", pre=["s_waitcnt lgkmcnt(0)"], slots=vs0)
        # step 2t+1 (parity 1)
        # the next item's Q rows: piece S_IT of this wavefront's 12 (1 KB each), straight into
        # the Q area (LDS DMA at m0), requested before the tile's pieces so that the wait at the
        # barrier (vmcnt(4)) leaves exactly those in flight
        pf = [
            f"s_cmp_lt_u32 {S_IT}, %[npf]",
            f"s_cbranch_scc0 LNQ{it}_%=",
            f"s_lshl_b32 {S_TMP}, {S_IT}, 10",
            f"s_add_u32 {S_TMP}, {S_TMP}, %[qlds]",
            f"s_mov_b32 m0, {S_TMP}",
            f"s_mul_i32 {S_TMP}, {S_IT}, %[qstep]",
            f"v_add_u32 {vr(QV)}, {S_TMP}, {vr(QVOFF)}",
            "s_nop 0",
            f"buffer_load_dwordx4 {vr(QV)}, {SRD_Q}, 0 offen lds",
            f"LNQ{it}_%=:",
        ]
        self.phase(1, 0, f"0P1{it}", slots={1: pf + ld, 2: adv})
        if self.nb == 3:
            self.phase(1, 1, f"1P1{it}", pre=["s_waitcnt lgkmcnt(0)"], slots=ks1)
            self.phase(1, 2, f"2P1{it}", slots=vs1)
        else:
            self.phase(1, 1, f"1P1{it}", pre=["s_waitcnt lgkmcnt(0)"], slots=vs1)
        e("s_waitcnt vmcnt(4) lgkmcnt(0)")  # tile t+2 in LDS (and this wavefront's reads done)
        e("s_barrier")
        e(f"s_add_u32 {S_IT}, {S_IT}, 1")

    def build(self):
        e = self.emit
        # ---- prologue: first operands, zero state, scores of step 0 for every block and the
        # running max taken from them ----
        for ks in range(4):
            e(f"ds_read_b128 {ar(KB(0, ks), 4)}, {vr(KL + ks)}")
            e(f"ds_read_b128 {ar(KB(1, ks), 4)}, {vr(KL + ks)} offset:{HALF_BYTES}")
        for ch in range(2):
            for db in range(2):
                off = V_BASE + ch * 16 * ROW_BYTES
                e(f"ds_read_b64_tr_b16 {ar(VB(0, ch, db), 2)}, {vr(VL + 2 * db)} offset:{off}")
                e(f"ds_read_b64_tr_b16 {ar(VB(0, ch, db) + 2, 2)}, {vr(VL + 2 * db + 1)} offset:{off}")
        for i in range(16):
            e(f"v_accvgpr_write_b32 {ar(VB(1, 0, 0) + i)}, 0")
        for i in range(8):
            e(f"v_mov_b32 {vr(P(self.nb - 1) + i)}, 0")
        for i in range(96):
            e(f"v_accvgpr_write_b32 {ar(i)}, 0")
        for b in range(self.nb):
            e(f"v_mov_b32 {vr(LRUN(b))}, 0")
        e("s_waitcnt lgkmcnt(0)")
        for b in range(self.nb):
            for ks in range(4):
                c = "0" if ks == 0 else vr(S(b), 16)
                e(f"{self.mfma} {vr(S(b), 16)}, {ar(KB(0, ks), 4)}, {ar(Q(b, ks), 4)}, {c}")
        # tile 2 requested (tile t+3 is requested during tile t)
        e(f"s_mov_b32 {S_BUFC}, {2 * TILE_BYTES}")
        for x in self.tile_dma() + self.advance():
            e(x)
        e(f"v_mov_b32 {vr(NEGINF)}, 0xff800000")
        # the running max of each block = the true max of its step-0 scores: the score chains
        # start from -max; the scores of blocks 0 .. nb-2 are shifted here, those of the last
        # block are computed again by step 0's first phase from the new chain start
        for b in range(self.nb):
            if b in (0, self.nb - 1):
                e("s_nop 7")  # (the scores' MFMAs were issued just before)
                e("s_nop 7")
            for x in self.row_max(b, RT):
                e(x)
            e(f"v_mov_b32 {vr(MRUN(b))}, {vr(RT)}")
            for i in range(16):
                e(f"v_sub_f32 {vr(CINIT(b) + i)}, 0, {vr(RT)}")
            if b < self.nb - 1:
                for i in range(16):
                    e(f"v_sub_f32 {vr(S(b) + i)}, {vr(S(b) + i)}, {vr(RT)}")
        e(f"s_mov_b32 {S_LIMIT}, {SUM_LIMIT}")
        e(f"s_mov_b32 {S_IT}, 0")
        e("s_cmp_eq_u32 %[n], 0")
        e("s_cbranch_scc1 LEND_%=")
        # ---- loop over tiles, two per trip ----
        e("LLOOP_%=:")
        self.iteration("A")
        e(f"s_cmp_ge_u32 {S_IT}, %[n]")
        e("s_cbranch_scc1 LEND_%=")
        self.iteration("B")
        e(f"s_cmp_lt_u32 {S_IT}, %[n]")
        e("s_cbranch_scc1 LLOOP_%=")
        e("LEND_%=:")
        e("s_waitcnt vmcnt(0) lgkmcnt(0)")
        # ---- tail: the r = n_sub - 2 n remaining steps (0, 1 or 2; the last one masked) ----
        # state: S(s_end) of blocks 0 and 1, P(s_end - 1) of block 2, K(s_end) and K(s_end + 1) in
        # K buffers 0 and 1, V(s_end - 1) and V(s_end) in V buffers 1 and 0
        e("s_cmp_eq_u32 %[r], 0")
        e("s_cbranch_scc1 LT0_%=")
        e("s_cmp_eq_u32 %[r], 1")
        e("s_cbranch_scc1 LT1_%=")
        # r = 2: step s_end (full), then step s_end + 1 (masked); V(s_end + 1) -> V buffer 1
        e(f"s_and_b32 {S_TMP}, {S_IT}, 3")
        e(f"s_mul_i32 {S_TMP}, {S_TMP}, {TILE_BYTES}")
        for i in range(4):
            e(f"v_add_u32 {vr(VADDRT + i)}, {S_TMP}, {vr(VL + i)}")
        tvr = self.v_reads(0, base=VADDRT)
        tslots = {1: tvr[0:2], 2: tvr[2:4], 3: tvr[4:6], 4: tvr[6:8]}
        nb = self.nb
        for ph in range(nb):
            pre = ["s_waitcnt lgkmcnt(0)"] if ph == 1 else []
            self.phase(0, ph, f"{ph}T2", pre=pre, slots=tslots if ph == nb - 1 else None)
        e("s_waitcnt lgkmcnt(0)")
        for ph in range(nb):
            self.phase(1, ph, f"{ph}T2b", do_s=ph == 0, mask=True)
        self.final_pv(1)
        e("s_branch LTEND_%=")
        # r = 1: step s_end, masked
        e("LT1_%=:")
        for ph in range(nb):
            pre = ["s_waitcnt lgkmcnt(0)"] if ph == 1 else []
            self.phase(0, ph, f"{ph}T1", pre=pre, do_s=ph == 0, mask=True)
        self.final_pv(0)
        e("s_branch LTEND_%=")
        # r = 0: only the last block's last P V
        e("LT0_%=:")
        self.final_pv(1)
        e("LTEND_%=:")
        e("s_nop 7")
        e("s_nop 7")
        e("s_nop 7")
        e("s_branch LDONE_%=")
        self.out.extend(self.rare)
        e("LDONE_%=:")
        e("s_nop 4")
        return self.out


def _vregs(ops):
    out = set()
    for o in ops:
        o = o.rstrip(",")
        if o.startswith("v["):
            lo, hi = o[2:-1].split(":")
            out |= set(range(int(lo), int(hi) + 1))
        elif o[:1] == "v" and o[1:].isdigit():
            out.add(int(o[1:]))
    return out


def check_trans_hazards(body):
    """A transcendental's result is not forwarded: the VALU instruction right after a v_exp must
    not read it (one wait state)."""
    for i in range(len(body) - 1):
        if body[i].startswith("v_exp"):
            dst = _vregs(body[i].split()[1:2])
            nxt = body[i + 1].split()
            if nxt and nxt[0].startswith("v_") and dst & _vregs(nxt[2:]):
                raise AssertionError(f"trans hazard: {body[i]!r} -> {body[i + 1]!r}")


def render() -> str:
    lines = [
        "// Generated by gen_dense_loop.py -- do not edit; edit the generator and rebuild.",
        "// The main loop of dense_pipe_kernel (attn_dense.hip); see the generator for the design.",
        "#pragma once",
        "",
    ]
    for dtype in ("bf16", "f16"):
        for nb in (3, 2):
            body = Gen(dtype, nb).build()
            check_trans_hazards(body)
            suffix = "" if nb == 3 else "_NB2"
            lines.append(f"#define WDRZ_DENSE_LOOP_{dtype.upper()}{suffix} \\")
            for s in body:
                lines.append(f'  "{s}\\n" \\')
            lines.append('  ""')
            lines.append("")
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    out = Path(sys.argv[1]) if len(sys.argv) > 1 else Path(__file__).with_name("dense_loop.inc")
    text = render()
    if not out.exists() or out.read_text() != text:
        out.write_text(text)
