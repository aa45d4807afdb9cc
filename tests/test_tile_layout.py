"""CPU model of the 256-row kernel's LDS tile layout (csrc/segment_tile.hip, Tile32 / Pipe32).

The kernel copies a 64-token tile of K ([d][token] rows of the pool) and V
([token][d] rows) into LDS with one 16-byte DMA slot per lane, and reads the
MFMA operands back with ds_read_b64_tr_b16: within each 16-lane group, lane
4a + b receives element b of the 8-byte chunks addressed by lanes a, a + 4,
a + 8 and a + 12.  This model restates the kernel's slot and offset formulas
and checks, for d = 32, 64 and 128:

  * the copy writes every slot of a block exactly once (a permutation);
  * every transposing read hands each lane exactly the (token, d) elements
    that the v_mfma_f32_32x32x16 operand layout asks for: the K operand of
    QK (lane l: token l % 32, d = 16 ks + 8 (l // 32) + j) and the V^T operand
    of PV (lane l: d = 32 dt + l % 32, token = 16 sub + 8 (j // 4) +
    4 (l // 32) + j % 4, the k order in which the QK result leaves P);
  * each 16-lane group reads one 128-byte run, and groups 0/1 and 2/3 land in
    opposite 128-byte halves of the 256-byte bank row (no bank conflicts).
"""
import pytest

BLK = 512  # elements (16-bit) per 1 KiB block


class Tile32:
    def __init__(self, d):
        self.D = d
        self.KBLK = d // 8
        self.VROWS = 512 // d
        self.VBLK = 64 // self.VROWS
        self.NDU = d // 16

    def vunit(self, rq, du):
        return ((rq * self.NDU + du) & ~1) | ((du ^ rq) & 1)

    def vrun(self, tau, du):
        return BLK * (self.KBLK + tau // self.VROWS) + 64 * self.vunit((tau % self.VROWS) >> 2, du)

    def vdelta(self, sb, sub, r, dt):
        return self.vrun(sb + 16 * sub + 8 * r, 2 * dt) - self.vrun(0, 0)

    # -- the copy: what pool element each LDS element of the tile holds
    def tile_contents(self):
        """dict: LDS element offset -> ('K', d, token) or ('V', token, d)."""
        D = self.D
        out = {}
        for blk in range(self.KBLK + self.VBLK):
            for lane in range(64):
                if blk < self.KBLK:
                    u = lane >> 4
                    h = ((lane >> 3) & 1) ^ (u & 1)
                    ch = 2 * u + ((lane >> 2) & 1)
                    j = 4 * h + (lane & 3)
                    for x in range(8):
                        out[blk * BLK + 8 * lane + x] = ("K", 8 * blk + j, 8 * ch + x)
                else:
                    uidx, sin = lane >> 3, lane & 7
                    lin_hi = uidx & ~1
                    rq = lin_hi // self.NDU
                    du = ((lin_hi % self.NDU) & ~1) | ((uidx & 1) ^ (rq & 1))
                    jr = 4 * rq + (sin & 3)
                    s = 2 * du + (sin >> 2)
                    tok = self.VROWS * (blk - self.KBLK) + jr
                    for x in range(8):
                        out[blk * BLK + 8 * lane + x] = ("V", tok, 8 * s + x)
        return out

    def lane_consts(self, lane):
        g, i = lane >> 4, lane & 15
                                                  # within a 128-byte run
        inn = 32 * ((i >> 1) & 1) + 8 * (i >> 2) + 4 * (i & 1)
        kof0 = BLK * (g >> 1) + 128 * (g & 1) + 64 * (g & 1) + inn
        kof1 = BLK * (g >> 1) + 128 * (g & 1) + 64 * (1 - (g & 1)) + inn
        vof = self.vrun(4 * (g >> 1), g & 1) + inn
        return kof0, kof1, vof


def tr_read(contents, addrs):
    """One ds_read_b64_tr_b16: addrs[l] is lane l's element offset (4 elements).
    Returns per lane the 4 elements it receives."""
    out = []
    for lane in range(64):
        grp, a, b = lane >> 4, (lane & 15) >> 2, lane & 3
        out.append([contents[addrs[16 * grp + a + 4 * e] + b] for e in range(4)])
    return out


def banks_ok(addrs):
    """Each 16-lane group reads one 128-byte run; groups 0/1 and 2/3 take opposite halves."""
    runs, halves = [], []
    for grp in range(4):
        byte = sorted(2 * addrs[16 * grp + x] for x in range(16))
        lo = byte[0]
        if lo % 128 or byte[-1] + 8 - lo != 128 or len({v // 8 for v in byte}) != 16:
            return False
        runs.append(lo)
        halves.append((lo // 128) % 2)
    return halves[0] != halves[1] and halves[2] != halves[3]


@pytest.mark.parametrize("d", [32, 64, 128])
def test_copy_fills_every_slot_once(d):
    t = Tile32(d)
    c = t.tile_contents()
    assert len(c) == (t.KBLK + t.VBLK) * BLK
    k = sorted(v[1:] for v in c.values() if v[0] == "K")
    v = sorted(v[1:] for v in c.values() if v[0] == "V")
    assert k == sorted((dd, tok) for dd in range(d) for tok in range(64))
    assert v == sorted((tok, dd) for tok in range(64) for dd in range(d))


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("sb", [0, 32])
def test_k_reads_give_the_qk_operand(d, sb):
    t = Tile32(d)
    c = t.tile_contents()
    for ks in range(d // 16):
        halves = []
        for h in range(2):
            addrs = [t.lane_consts(l)[h] + 2 * BLK * ks + 8 * sb for l in range(64)]
            assert banks_ok(addrs), (d, sb, ks, h)
            halves.append(tr_read(c, addrs))
        for lane in range(64):
            got = halves[0][lane] + halves[1][lane]
            want = [("K", 16 * ks + 8 * (lane // 32) + j, sb + lane % 32) for j in range(8)]
            assert got == want, (d, sb, ks, lane)


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("sb", [0, 32])
def test_v_reads_give_the_pv_operand(d, sb):
    t = Tile32(d)
    c = t.tile_contents()
    for dt in range(d // 32):
        for sub in range(2):
            runs = []
            for r in range(2):
                addrs = [t.lane_consts(l)[2] + t.vdelta(sb, sub, r, dt) for l in range(64)]
                assert banks_ok(addrs), (d, sb, dt, sub, r)
                runs.append(tr_read(c, addrs))
            for lane in range(64):
                got = runs[0][lane] + runs[1][lane]
                want = [("V", sb + 16 * sub + 8 * (j // 4) + 4 * (lane // 32) + j % 4, 32 * dt + lane % 32)
                        for j in range(8)]
                assert got == want, (d, sb, dt, sub, lane)


def test_vdelta_is_the_same_for_every_lane_group():
    for d in (32, 64, 128):
        t = Tile32(d)
        for g in range(4):
            for sb in (0, 32):
                for sub in range(2):
                    for r in range(2):
                        for dt in range(d // 32):
                            tau = sb + 16 * sub + 8 * r + 4 * (g >> 1)
                            direct = t.vrun(tau, 2 * dt + (g & 1))
                            assert direct == t.vrun(4 * (g >> 1), g & 1) + t.vdelta(sb, sub, r, dt)
