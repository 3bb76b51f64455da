"""GPU parity for the MoE and EXL3 parameter-block kinds of vybdq_launch_pblock: the reference's own
blocks (native/kernels/moe.vyb:15-19; native/kernels/exl3.vyb:264, exl3dq.vyb:8-11, exl3.vyb:318-321)
written to device memory and launched through the C-ABI, against the float64 oracle; invalid blocks
are reported and not computed; a captured graph replays with a rewritten block."""

import numpy as np
import pytest
import torch

from oracle import exl3, matmul, moe
from tests.conftest import GOLDEN
from vybforge_amd import _lib

pytestmark = pytest.mark.gpu

MH, MI, ME, MK = 4096, 2048, 288, 8


def status():
    return _lib.lib.vybdq_pblock_status()


def stream():
    return torch.cuda.current_stream().cuda_stream


def f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


# ---- MoE (moe.vyb) ----------------------------------------------------------------------------

class MoeBlock:
    """Device buffers and the 15-word block of one MoE fixture call (moe_driver.vyb:104-145)."""

    def __init__(self, dev, rng, S, y=None, G=None, bias=None, wscale=0.05):
        self.S = S
        self.y = y if y is not None else rng.standard_normal((S, MH)).astype(np.float32)
        self.G = G if G is not None else (rng.standard_normal((ME, MH)) * 0.03).astype(np.float32)
        self.bias = bias if bias is not None else (rng.standard_normal(ME) * 0.1).astype(np.float32)
        shapes = [(MH, MI), (MH, MI), (MI, MH), (MH, MI), (MH, MI), (MI, MH)]
        self.w = [(rng.standard_normal(s) * wscale).astype(np.float32) for s in shapes]
        self.d = dict(y=f32(self.y, dev), G=f32(self.G, dev), bias=f32(self.bias, dev))
        self.d["w"] = [f32(w, dev) for w in self.w]
        self.d["LG"] = torch.full((256, ME), -7.0, device=dev)
        self.d["IX"] = torch.full((256, MK), -7.0, device=dev)
        self.d["WT"] = torch.full((256, MK), -7.0, device=dev)
        self.d["AC"] = torch.full((256, 9, MI), -7.0, device=dev)
        self.d["out"] = torch.full((256, MH), -7.0, device=dev)
        self.words = np.zeros(15, np.int64)
        self.set_words(S)
        self.pb = torch.from_numpy(self.words.copy()).to(dev)

    def set_words(self, S, y=None):
        d = self.d
        self.words[:] = [(y if y is not None else d["y"]).data_ptr(), d["G"].data_ptr(), d["bias"].data_ptr(),
                         d["LG"].data_ptr(), d["IX"].data_ptr(), d["WT"].data_ptr(), d["AC"].data_ptr(),
                         *[w.data_ptr() for w in d["w"]], d["out"].data_ptr(), S]

    def launch(self):
        _lib.call("vybdq_launch_pblock", _lib.PB_MOE, self.pb.data_ptr(), stream())

    def oracle(self, y=None):
        return moe.fixture_block(self.y if y is None else y, self.G, self.bias, *self.w)


def check_moe(blk, S, y=None, untouched_from=None):
    lg, idx, w, act, out = blk.oracle(y)
    g_lg = blk.d["LG"][:S].cpu().numpy().astype(np.float64)
    # float64 sums in another order: the float32 logits agree to one ulp
    ulp = np.spacing(np.abs(lg).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(g_lg - lg) <= ulp), "logits"
    # routing from the kernel's own logits: identical ids and order, weights to float32 rounding
    ridx, rw = moe.fixture_route(g_lg.astype(np.float32), blk.bias)
    g_ix = blk.d["IX"][:S].cpu().numpy()
    assert np.array_equal(g_ix, ridx.astype(np.float32)), "expert ids"
    assert np.abs(blk.d["WT"][:S].cpu().numpy() - rw).max() < 1e-6, "weights"
    # activations and output against float64 (verify_moe_vyb.py:66-73 gates rel < 1e-5)
    g_ac = blk.d["AC"][:S].cpu().numpy()
    assert matmul.rel_maxnorm(g_ac, act) < 1e-6
    g_out = blk.d["out"][:S].cpu().numpy()
    assert matmul.rel_maxnorm(g_out, out) < 1e-5
    # untouched past S (past the largest S of earlier calls on the same buffers)
    u = S if untouched_from is None else untouched_from
    if u < 256:
        assert (blk.d["out"][u:] == -7.0).all() and (blk.d["AC"][u:] == -7.0).all()


@pytest.mark.parametrize("S", [1, 4, 16, 37, 256])
def test_pblock_moe(dev, S):
    blk = MoeBlock(dev, np.random.default_rng(100 + S), S)
    blk.launch()
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    check_moe(blk, S)


def test_pblock_moe_clamps_and_reference_routing(dev):
    """Large weights drive g and u past the +-10 clamps; the routing of the reference's own golden
    logits (moe_golden.npz, four tokens) comes out of the kernel unchanged: y carries the logits
    and G is the identity on the first 288 columns, so LG = float32(logit)."""
    z = np.load(f"{GOLDEN}/moe_golden.npz")
    S = z["logits"].shape[0]
    y = np.zeros((S, MH), np.float32)
    y[:, :ME] = z["logits"].astype(np.float32)
    y[:, ME:] = np.random.default_rng(5).standard_normal((S, MH - ME)).astype(np.float32)
    G = np.zeros((ME, MH), np.float32)
    G[np.arange(ME), np.arange(ME)] = 1.0
    blk = MoeBlock(dev, np.random.default_rng(6), S, y=y, G=G, bias=z["bias"].astype(np.float32), wscale=0.3)
    blk.launch()
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    ix = blk.d["IX"][:S].cpu().numpy().astype(np.int64)
    wt = blk.d["WT"][:S].cpu().numpy()
    for s in range(S):
        a, b = dict(zip(ix[s].tolist(), wt[s].tolist())), dict(zip(z["ref_idx"][s].tolist(), z["ref_w"][s].tolist()))
        assert set(a) == set(b) and max(abs(a[e] - b[e]) for e in a) < 1e-4
    _, _, _, act, _ = blk.oracle()
    assert np.abs(act).max() > 50.0  # the clamps were reached: |silu(10) * 10| ~ 100
    check_moe(blk, S)


def test_pblock_moe_rewritten_between_graph_replays(dev):
    """The block is read when the launch runs: a captured graph replayed after S and y were
    rewritten computes the new call."""
    rng = np.random.default_rng(11)
    blk = MoeBlock(dev, rng, 5)
    assert status() == 0  # the device's status word is set up before the capture
    y2 = rng.standard_normal((9, MH)).astype(np.float32)
    y2_d = f32(y2, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            _lib.call("vybdq_launch_pblock", _lib.PB_MOE, blk.pb.data_ptr(), s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    for S, y in [(5, None), (9, y2), (5, None)]:
        blk.set_words(S, None if y is None else y2_d)
        blk.pb.copy_(torch.from_numpy(blk.words.copy()))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert status() == 0, _lib.last_error()
        check_moe(blk, S, y, untouched_from=9)


def test_pblock_moe_invalid_blocks_are_reported(dev):
    blk = MoeBlock(dev, np.random.default_rng(12), 3)
    for S in (0, 257):
        blk.set_words(S)
        blk.pb.copy_(torch.from_numpy(blk.words.copy()))
        blk.launch()
        assert status() == _lib.ERR_SHAPE and "MoE" in _lib.last_error()
        assert status() == 0  # cleared
    blk.set_words(3)
    blk.words[9] = 0  # no down matrix
    blk.pb.copy_(torch.from_numpy(blk.words.copy()))
    blk.launch()
    assert status() == _lib.ERR_SHAPE
    assert (blk.d["out"] == -7.0).all() and (blk.d["LG"] == -7.0).all()


# ---- EXL3 fused decode + column transform (exl3dq1 / exl3dq1s) and exl3inv ------------------

class Exl3Block:
    def __init__(self, dev, rng, rows, cw, H):
        self.rows, self.cw = rows, cw
        self.q = rng.integers(0, 256, (rows // 16) * (cw // 16) * 128, dtype=np.uint8).tobytes()
        self.body = exl3.tile_map_bytes()
        hdr = np.array([cw, (rows // 16) * (cw // 16)], "<i8").tobytes()
        td = np.frombuffer(hdr + self.body + bytes(1024), np.uint8)
        self.td = torch.from_numpy(td.copy()).to(dev)
        self.q_d = torch.from_numpy(np.frombuffer(self.q, np.uint8).copy()).to(dev)
        self.H = np.asarray(H, np.float32)
        self.H_d = f32(self.H, dev)
        self.T = torch.full((rows * cw,), -7.0, device=dev)
        inv = self.td.data_ptr() + 16 + 4096
        self.pb = torch.tensor([self.q_d.data_ptr(), self.td.data_ptr(), self.H_d.data_ptr(), self.T.data_ptr(), cw, inv],
                               dtype=torch.int64, device=dev)
        self.pb_inv = torch.tensor([self.td.data_ptr(), 4096], dtype=torch.int64, device=dev)

    def build_inverse(self):
        _lib.call("vybdq_launch_pblock", _lib.PB_EXL3INV, self.pb_inv.data_ptr(), stream())

    def launch(self, grid=None, block=256):
        grid = grid if grid is not None else self.rows * self.cw // block
        _lib.call("vybdq_launch_pblock_grid", _lib.PB_EXL3DQ, self.pb.data_ptr(), grid, block, stream())

    def what(self):
        return exl3.map_decode_f32(self.q, self.rows, self.cw, self.body, exl3.tile_map_inverse(self.body))


def test_pblock_exl3inv_builds_the_inverse_map(dev):
    blk = Exl3Block(dev, np.random.default_rng(1), 128, 128, np.eye(128))
    blk.build_inverse()
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    inv = blk.td[16 + 4096:].cpu().numpy().view(np.uint32)
    assert np.array_equal(inv, exl3.tile_map_inverse(blk.body))


@pytest.mark.parametrize("rows,cw", [(128, 128), (128, 256), (384, 384)])
def test_pblock_exl3dq_identity_is_the_decode(dev, rows, cw):
    """H = I: the transform is exact, so T is the map-decoded What bit for bit (in T order)."""
    blk = Exl3Block(dev, np.random.default_rng(rows + cw), rows, cw, np.eye(128))
    blk.build_inverse()
    blk.launch()
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    ref = exl3.column_transform_f64(blk.what(), np.eye(128))
    assert np.array_equal(blk.T.cpu().numpy().astype(np.float64), ref)


@pytest.mark.parametrize("H", ["random", "hadamard"])
def test_pblock_exl3dq_transform(dev, H):
    rows, cw = 256, 512
    rng = np.random.default_rng(21)
    Hm = rng.standard_normal((128, 128)) if H == "random" else exl3.hadamard128() / np.sqrt(128.0)
    blk = Exl3Block(dev, rng, rows, cw, Hm)
    blk.build_inverse()
    blk.launch()
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    ref = exl3.column_transform_f64(blk.what(), blk.H.astype(np.float64))
    got = blk.T.cpu().numpy()
    # 128-term float32 fma chains against float64
    assert matmul.rel_maxnorm(got, ref) < 1e-5


def test_pblock_exl3dq_glm_shape_slice(dev):
    """K = 2048 rows x N = 4096 columns (the down_proj fixture the map was made for,
    gen_map_bin.py:17-18): every block is computed; two blocks are checked against float64."""
    rows, cw = 2048, 4096
    rng = np.random.default_rng(22)
    Hm = exl3.hadamard128() / np.sqrt(128.0)
    blk = Exl3Block(dev, rng, rows, cw, Hm)
    blk.build_inverse()
    blk.launch(block=512)
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    T = blk.T.cpu().numpy()
    assert not (T == -7.0).any()
    q = np.frombuffer(blk.q, np.uint8).reshape(rows // 16, cw // 16, 128)
    inv = exl3.tile_map_inverse(blk.body)
    for kb, nb in [(0, 0), (15, 31)]:
        sub = q[kb * 8:(kb + 1) * 8, nb * 8:(nb + 1) * 8].tobytes()
        what = exl3.map_decode_f32(sub, 128, 128, blk.body, inv)
        ref = what.astype(np.float64) @ Hm
        off = (kb * (cw // 128) + nb) * 16384
        assert matmul.rel_maxnorm(T[off:off + 16384].reshape(128, 128), ref) < 1e-5


def test_pblock_exl3dq_invalid_blocks_are_reported(dev):
    blk = Exl3Block(dev, np.random.default_rng(3), 128, 128, np.eye(128))
    blk.build_inverse()
    torch.cuda.synchronize()
    assert status() == 0
    blk.launch(grid=blk.rows * blk.cw // 256 - 1)  # not rows x cw threads
    assert status() == _lib.ERR_SHAPE and "EXL3" in _lib.last_error()
    words = blk.pb.cpu().numpy().copy()
    words[4] = 100  # cw not a multiple of 128
    blk.pb.copy_(torch.from_numpy(words))
    blk.launch(grid=128 * 100 // 64, block=64)
    assert status() == _lib.ERR_SHAPE
    words[4] = 128
    blk.pb.copy_(torch.from_numpy(words))
    bad = blk.td.cpu().numpy().copy()
    bad[16 + 16 * 3 + 1] = 1  # slot 3's first nibble index becomes 256 + ...
    blk.td.copy_(torch.from_numpy(bad))
    blk.launch()
    assert status() == _lib.ERR_SHAPE
    assert (blk.T == -7.0).all()
    with pytest.raises(_lib.VybdqError):
        _lib.call("vybdq_launch_pblock", _lib.PB_EXL3DQ, blk.pb.data_ptr(), stream())


# ---- the stages of the separate EXL3 reconstruction: exl3deq(32), exl3hgen(32), exl3had1(32),
# exl3had2(32), exl3cvt32 (exl3.vyb:36-256), as glm_engine.vyb:1103-1200 and
# native/host/glm_exl3_check32.vyb:150-240 chain them -------------------------------------------

PREC = {"f64": (np.float64, torch.float64, _lib.F64), "f32": (np.float32, torch.float32, _lib.F32)}
HGEN = {"f64": _lib.PB_EXL3HGEN, "f32": _lib.PB_EXL3HGEN32}
HAD1 = {"f64": _lib.PB_EXL3HAD1, "f32": _lib.PB_EXL3HAD132}
HAD2 = {"f64": _lib.PB_EXL3HAD2, "f32": _lib.PB_EXL3HAD232}


def pblock(words, dev):
    return torch.tensor([int(w) for w in words], dtype=torch.int64, device=dev)


def launch(kind, pb):
    _lib.call("vybdq_launch_pblock", kind, pb.data_ptr(), stream())


def map_tab(dev, cw, ntiles, body=None):
    body = exl3.tile_map_bytes() if body is None else body
    hdr = np.array([cw, ntiles], "<i8").tobytes()
    return torch.from_numpy(np.frombuffer(hdr + body, np.uint8).copy()).to(dev)


def half_scales(rng, n):
    return (np.abs(rng.standard_normal(n)) * 0.12 + 0.02).astype(np.float16)


@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_pblock_exl3hgen_bit_exact(dev, prec):
    npd, td, _ = PREC[prec]
    H = torch.full((128, 128), -7.0, dtype=td, device=dev)
    launch(HGEN[prec], pblock([H.data_ptr()], dev))
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    assert np.array_equal(H.cpu().numpy(), exl3.hgen(npd))


@pytest.mark.parametrize("prec", ["f64", "f32"])
@pytest.mark.parametrize("rows,cw", [(16, 16), (64, 256), (2048, 4096)])
def test_exl3_deq_map_bit_exact(dev, prec, rows, cw):
    """exl3deq / exl3deq32 through vybdq_exl3_deq_map: every value bit-exact (the half sum is exact
    in float32), every position written once; 2048 x 4096 is the down_proj the map was made for."""
    npd, td, dt = PREC[prec]
    rng = np.random.default_rng(rows + cw)
    ntiles = (rows // 16) * (cw // 16)
    q = rng.integers(0, 256, ntiles * 128, dtype=np.uint8).tobytes()
    q_d = torch.from_numpy(np.frombuffer(q, np.uint8).copy()).to(dev)
    tab = map_tab(dev, cw, ntiles)
    o = torch.full((rows, cw), -7.0, dtype=td, device=dev)
    _lib.call("vybdq_exl3_deq_map", q_d.data_ptr(), tab.data_ptr(), o.data_ptr(), dt, stream())
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    ref = exl3.map_deq(q, exl3.tile_map_bytes(), cw, ntiles).astype(npd)
    assert np.array_equal(o.cpu().numpy(), ref)


@pytest.mark.parametrize("prec", ["f64", "f32"])
@pytest.mark.parametrize("nbc_full", [True, False])
def test_pblock_exl3had1(dev, prec, nbc_full):
    npd, td, _ = PREC[prec]
    rng = np.random.default_rng(31)
    rows, cw = 256, 512
    nbc = cw // 128 if nbc_full else 2
    nblocks = rows // 128 * nbc
    W = rng.standard_normal((rows, cw)).astype(npd)
    H = exl3.hgen(npd)
    W_d, H_d = torch.from_numpy(W).to(dev), torch.from_numpy(H).to(dev)
    T = torch.full((rows * cw,), -7.0, dtype=td, device=dev)
    launch(HAD1[prec], pblock([W_d.data_ptr(), T.data_ptr(), H_d.data_ptr(), cw, nbc, nblocks], dev))
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    ref = exl3.had1_f64(W, H, cw, nbc, nblocks)
    got = T.cpu().numpy()
    # 128-term fma chains against float64 sums in another order
    assert matmul.rel_maxnorm(got[:nblocks * 16384], ref) < (1e-13 if prec == "f64" else 1e-5)
    assert (got[nblocks * 16384:] == -7.0).all()


@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_pblock_exl3had2(dev, prec):
    npd, td, _ = PREC[prec]
    rng = np.random.default_rng(32)
    rows, cw = 256, 384
    nbc, nblocks = cw // 128, rows // 128 * (cw // 128)
    tmp = rng.standard_normal(nblocks * 16384).astype(npd)
    H = exl3.hgen(npd)
    su, sv = half_scales(rng, rows), half_scales(rng, cw)
    d = [torch.from_numpy(a).to(dev) for a in (tmp, H, su, sv)]
    O = torch.full((rows, cw), -7.0, dtype=td, device=dev)
    launch(HAD2[prec], pblock([d[0].data_ptr(), O.data_ptr(), d[1].data_ptr(), d[2].data_ptr(), d[3].data_ptr(),
                               cw, nbc, nblocks], dev))
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    ref = exl3.had2_f64(tmp, H, su, sv, cw, nbc, nblocks)
    assert matmul.rel_maxnorm(O.cpu().numpy(), ref) < (1e-13 if prec == "f64" else 1e-5)


@pytest.mark.parametrize("n", [1, 1000003])
def test_pblock_exl3cvt32_bit_exact(dev, n):
    rng = np.random.default_rng(n)
    S = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(dev)
    D = torch.full((n + 5,), -7.0, dtype=torch.float64, device=dev)
    launch(_lib.PB_EXL3CVT32, pblock([S.data_ptr(), D.data_ptr(), n], dev))
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    assert torch.equal(D[:n], S.double()) and (D[n:] == -7.0).all()


def exl3_matrix(rng, rows, cw):
    ntiles = (rows // 16) * (cw // 16)
    q = rng.integers(0, 256, ntiles * 128, dtype=np.uint8).tobytes()
    su, sv = half_scales(rng, rows), half_scales(rng, cw)
    ref = exl3.rotate_blocks(exl3.map_deq(q, exl3.tile_map_bytes(), cw, ntiles), su, sv)
    return q, su, sv, ref


@pytest.mark.parametrize("prec", ["f64", "f32"])
def test_exl3_separate_pipeline_matches_the_rotation(dev, prec):
    """deq -> hgen -> had1 -> had2 (-> cvt32 for the f32 chain), glm_exl3_check32.vyb:150-240 with
    the f64 or the f32 kernels: the float64 result equals the oracle's rotated dequant."""
    npd, td, dt = PREC[prec]
    rng = np.random.default_rng(33)
    rows, cw = 256, 512
    q, su, sv, ref = exl3_matrix(rng, rows, cw)
    ntiles, nbc = (rows // 16) * (cw // 16), cw // 128
    nblocks = rows // 128 * nbc
    q_d = torch.from_numpy(np.frombuffer(q, np.uint8).copy()).to(dev)
    tab = map_tab(dev, cw, ntiles)
    od = torch.empty((rows, cw), dtype=td, device=dev)
    H = torch.empty((128, 128), dtype=td, device=dev)
    tmp = torch.empty((rows * cw,), dtype=td, device=dev)
    fd = torch.empty((rows, cw), dtype=td, device=dev)
    su_d, sv_d = torch.from_numpy(su).to(dev), torch.from_numpy(sv).to(dev)
    _lib.call("vybdq_exl3_deq_map", q_d.data_ptr(), tab.data_ptr(), od.data_ptr(), dt, stream())
    launch(HGEN[prec], pblock([H.data_ptr()], dev))
    launch(HAD1[prec], pblock([od.data_ptr(), tmp.data_ptr(), H.data_ptr(), cw, nbc, nblocks], dev))
    launch(HAD2[prec], pblock([tmp.data_ptr(), fd.data_ptr(), H.data_ptr(), su_d.data_ptr(), sv_d.data_ptr(),
                               cw, nbc, nblocks], dev))
    if prec == "f32":
        out = torch.empty((rows, cw), dtype=torch.float64, device=dev)
        launch(_lib.PB_EXL3CVT32, pblock([fd.data_ptr(), out.data_ptr(), rows * cw], dev))
    else:
        out = fd
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    assert matmul.rel_maxnorm(out.cpu().numpy(), ref) < (1e-12 if prec == "f64" else 1e-5)


def test_exl3_fused_pipeline_matches_the_rotation(dev):
    """exl3dq1s (decode + column transform) -> exl3had232 -> exl3cvt32, the exl3_deq32 chain of
    glm_engine.vyb:1103-1200, at the down_proj shape 2048 x 4096: float64 out vs the oracle."""
    rng = np.random.default_rng(34)
    rows, cw = 2048, 4096
    nbc, nblocks = cw // 128, rows // 128 * (cw // 128)
    blk = Exl3Block(dev, rng, rows, cw, np.zeros((128, 128)))
    launch(_lib.PB_EXL3HGEN32, pblock([blk.H_d.data_ptr()], dev))  # H / sqrt(128) into the block's H
    su, sv = half_scales(rng, rows), half_scales(rng, cw)
    ref = exl3.rotate_blocks(exl3.map_deq(blk.q, blk.body, cw, (rows // 16) * (cw // 16)), su, sv)
    blk.build_inverse()
    blk.launch(block=256)
    fd = torch.empty((rows, cw), dtype=torch.float32, device=dev)
    su_d, sv_d = torch.from_numpy(su).to(dev), torch.from_numpy(sv).to(dev)
    launch(_lib.PB_EXL3HAD232, pblock([blk.T.data_ptr(), fd.data_ptr(), blk.H_d.data_ptr(), su_d.data_ptr(),
                                       sv_d.data_ptr(), cw, nbc, nblocks], dev))
    out = torch.empty((rows, cw), dtype=torch.float64, device=dev)
    launch(_lib.PB_EXL3CVT32, pblock([fd.data_ptr(), out.data_ptr(), rows * cw], dev))
    torch.cuda.synchronize()
    assert status() == 0, _lib.last_error()
    assert matmul.rel_maxnorm(out.cpu().numpy(), ref) < 1e-5


def test_exl3_stage_invalid_blocks_are_reported(dev):
    """Stage blocks or maps that violate the preconditions write nothing and are reported."""
    rng = np.random.default_rng(35)
    W = torch.from_numpy(rng.standard_normal((128, 256)).astype(np.float32)).to(dev)
    H = torch.from_numpy(exl3.hgen(np.float32)).to(dev)
    T = torch.full((128 * 256,), -7.0, device=dev)
    su = torch.ones(256, dtype=torch.float16, device=dev)
    cases = [
        (_lib.PB_EXL3HAD132, [W.data_ptr(), T.data_ptr(), H.data_ptr(), 256, 0, 2]),        # nbc = 0
        (_lib.PB_EXL3HAD132, [W.data_ptr(), T.data_ptr(), H.data_ptr(), 256, 3, 3]),        # 128 nbc > cw
        (_lib.PB_EXL3HAD132, [W.data_ptr() + 4, T.data_ptr(), H.data_ptr(), 256, 2, 2]),    # misaligned W
        (_lib.PB_EXL3HAD232, [W.data_ptr(), T.data_ptr(), H.data_ptr(), su.data_ptr() + 1, su.data_ptr(), 256, 2, 2]),
        (_lib.PB_EXL3HAD232, [W.data_ptr(), T.data_ptr(), H.data_ptr(), su.data_ptr(), su.data_ptr(), 256, 2, 0]),
        (_lib.PB_EXL3CVT32, [W.data_ptr(), T.data_ptr(), -1]),                              # n < 0
        (_lib.PB_EXL3CVT32, [W.data_ptr(), T.data_ptr() + 4, 16]),                          # D not 8-aligned
        (_lib.PB_EXL3HGEN, [T.data_ptr() + 4]),                                               # H f64 misaligned
    ]
    for kind, words in cases:
        launch(kind, pblock(words, dev))
        assert status() == _lib.ERR_SHAPE, (hex(kind), words)
        assert (T == -7.0).all()
    # a map entry whose nibble index leaves the tile, and a cw that is not a multiple of 16
    q = torch.zeros(2 * 128, dtype=torch.uint8, device=dev)
    o = torch.full((16, 32), -7.0, device=dev)
    body = bytearray(exl3.tile_map_bytes())
    body[16 * 5 + 1] = 1
    for tab in (map_tab(dev, 32, 2, bytes(body)), map_tab(dev, 24, 2)):
        _lib.call("vybdq_exl3_deq_map", q.data_ptr(), tab.data_ptr(), o.data_ptr(), _lib.F32, stream())
        assert status() == _lib.ERR_SHAPE
        assert (o == -7.0).all()
