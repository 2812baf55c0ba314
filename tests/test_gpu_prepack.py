"""prepackWeights on the GPU: the packed s8 weight (TensorLayout PackedBHip)
gives bit-for-bit the result of the raw weight on every route (GEMV, small-M
MFMA, ring GEMM, split K), for [K,N] and [N,K] raw forms, with the precomputed
column sums standing in for the per-call pass (u8 A, A zero points), and
through the fp-activation and dequantizing routes; and the packed q4_1
weight with blocks along N (two planes) gives bit-for-bit the raw weight's
result on the ring route, the same up to f32 summation order on the GEMV
(which walks the planes in groups of 8 rows), within the Q4_1 tolerance
elsewhere (the skinny MFMA route of 3..48 rows)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce, norm_err

pytestmark = pytest.mark.gpu


def packed_skinny(M, K, a_f16):
    """The packed q4_1 planes' skinny MFMA route: f16 A, 3 <= M <= 48, K % 256 == 0."""
    return a_f16 and 3 <= M <= 48 and K % 256 == 0


def run(op, a_t, w_t, out_dtype, shape):
    import torch
    c = torch.zeros(shape, dtype=out_dtype, device="cuda")
    assert op.compute([na.tensor(c)], [a_t, w_t]) == na.OK
    torch.cuda.synchronize()
    return host(c)


@pytest.mark.parametrize("M,K,N", [(1, 4096, 1008), (3, 640, 200), (16, 1024, 512), (100, 512, 333),
                                   (512, 4096, 1024), (333, 2048, 512), (5, 100, 37)])
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("u8", [False, True])
def test_matmul_prepacked_matches_raw(M, K, N, trans_b, u8):
    import torch
    announce(f"prepack matmul {M}x{K}x{N} tb={trans_b} u8={u8}")
    seed = M + K + N + 2 * trans_b + 4 * u8
    a = dg.ints(seed, (M, K), 0, 255, np.uint8) if u8 else dg.act_s8(seed, (M, K))
    b = dg.ints(seed + 1, (N, K) if trans_b else (K, N), -127, 127)
    sb = dg.uniform(seed + 2, (N,), 0.001, 0.01)
    zp_a = 128 if u8 else 3
    op = na.MatMul(output_dtype=na.DT_S8, transpose_b=trans_b, act=na.EP_RELU)
    wt = na.tensor(dev(b), scale_data=sb, granularity=2)
    buf, packed = op.prepack(wt)
    assert packed is not None and packed.layout == na.LAYOUT_PACKED_B_HIP
    at = na.tensor(dev(a), scale=0.02, zero_point=zp_a)
    got_p = run(op, at, packed, torch.int8, (M, N))
    got_r = run(op, at, wt, torch.int8, (M, N))
    np.testing.assert_array_equal(got_p, got_r)
    # and against the oracle with an output scale
    c = torch.zeros((M, N), dtype=torch.int8, device="cuda")
    assert op.compute([na.tensor(c, scale=0.05)], [at, packed]) == na.OK
    torch.cuda.synchronize()
    want = oracle.gemm_i8(a, b, trans_b=trans_b, out_kind=oracle.OUT_S8, s_a=0.02, zp_a=zp_a, s_b=sb,
                          s_out=0.05, act=oracle.ACT_RELU)
    np.testing.assert_array_equal(host(c), want)


@pytest.mark.parametrize("M", [1, 16, 300])
def test_linear_prepacked_s32_and_f16(M):
    import torch
    announce(f"prepack linear M={M}")
    K, N = 1536, 384
    x = dg.act_s8(70 + M, (M, K))
    w = dg.ints(71, (N, K), -127, 127)
    for odt, tdt, ok in ((na.DT_S32, torch.int32, oracle.OUT_S32), (na.DT_F16, torch.float16, oracle.OUT_F16)):
        op = na.Linear(output_dtype=odt)
        wt = na.tensor(dev(w), scale=0.004)
        _, packed = op.prepack(wt)
        got = run(op, na.tensor(dev(x), scale=0.02), packed, tdt, (M, N))
        want = oracle.gemm_i8(x, w, trans_b=True, out_kind=ok, s_a=0.02, s_b=0.004)
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_matmul_fp_activation_prepacked():
    import torch
    announce("prepack fp-A matmul")
    M, K, N = 24, 1024, 256
    a = dg.normal(81, (M, K), 2.0).astype(np.float16)
    b = dg.ints(82, (K, N), -127, 127)
    s_a = dg.uniform(83, (M,), 0.01, 0.03)
    zp_a = dg.ints(84, (M,), -5, 5, np.int32)
    op = na.MatMul()
    _, packed = op.prepack(na.tensor(dev(b), scale=0.003))
    at = na.tensor(dev(a), scale_data=s_a, zero_point_data=zp_a, granularity=1)
    got = run(op, at, packed, torch.float16, (M, N))
    aq = oracle.quantize_linear(a, s_a, zp_a, axis=-1)
    want = oracle.gemm_i8(aq, b, out_kind=oracle.OUT_F16, s_a=s_a, zp_a=zp_a, s_b=0.003)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_prepack_rejects_mismatched_buffer_and_k():
    import torch
    announce("prepack rejects")
    K, N = 256, 64
    b = dg.ints(91, (K, N), -127, 127)
    op = na.MatMul(output_dtype=na.DT_S32)
    _, packed = op.prepack(na.tensor(dev(b)))
    # an A whose K needs a larger blob than this one
    a = dg.act_s8(92, (4, 512))
    c = torch.zeros((4, N), dtype=torch.int32, device="cuda")
    assert op.compute([na.tensor(c)], [na.tensor(dev(a)), packed]) == na.INVALID_ARGUMENT


@pytest.mark.parametrize("M,K,N,a_f16", [(1, 4096, 1000, True), (2, 1024, 300, True), (40, 4096, 2048, True),
                                         (300, 1024, 1000, True), (129, 192, 384, True), (3, 512, 256, False),
                                         (130, 1000, 200, False), (17, 512, 256, False)])
def test_matmul_q4_1_prepacked_matches_raw(M, K, N, a_f16):
    import torch
    announce(f"prepack q4_1 {M}x{K}x{N} f16={a_f16}")
    seed = 7 * M + K + N
    a = dg.normal(seed, (M, K)).astype(np.float16 if a_f16 else np.float32)
    blk = dg.q4_1_blocks(seed + 1, K, N)                 # [K][N/32] blocks
    op = na.MatMul(transpose_b=False)
    wt = na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[K, N])
    buf, packed = op.prepack(wt)
    assert packed is not None and packed.layout == na.LAYOUT_PACKED_B_HIP and packed.dtype == na.DT_Q4_1
    at = na.tensor(dev(a))
    got_p = run(op, at, packed, torch.float32, (M, N))
    got_r = run(op, at, wt, torch.float32, (M, N))
    if ((M > 2 and a_f16) or M > 16) and not packed_skinny(M, K, a_f16):
        # the f16 ring or the f32 MFMA GEMM: same decode, same order
        np.testing.assert_array_equal(got_p, got_r)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=False)
    scale = max(np.max(np.abs(want)), np.sqrt(np.mean(want ** 2)))
    err = float(np.max(np.abs(got_p - want)) / scale)
    assert err <= 2e-3, err
    # the GEMVs differ: the planes' kernel sums f32 products, the raw rows'
    # one-launch kernel dots f16 (a d) pairs, so each meets the oracle's bar
    err_r = float(np.max(np.abs(got_r - want)) / scale)
    assert err_r <= 2e-3, err_r


@pytest.mark.parametrize("M,K,N", [(5, 1000, 77), (64, 96, 40), (64, 256, 200), (3, 64, 200), (3, 37, 72),
                                   (1, 97, 40)])
def test_matmul_q4_1_prepacked_ragged_k(M, K, N):
    """Ragged shapes. K % 64 != 0 with M > 2 and no GEMV pass (K % 8 != 0 or
    M > 12): the packed weight and the raw one both take the generic MFMA
    kernel (the same decode and order, so the same bits). N = 200 (7 blocks
    per row): the packed weight takes the GEMV passes (M <= 12) or the ring.
    All within the Q4_1 tolerance of the oracle."""
    import torch
    announce(f"prepack q4_1 ragged {M}x{K}x{N}")
    a = dg.normal(M + K, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(N + K, K, N)
    op = na.MatMul(transpose_b=False)
    wt = na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[K, N])
    _, packed = op.prepack(wt)
    got = run(op, na.tensor(dev(a)), packed, torch.float32, (M, N))
    if M > 2 and K % 64 and (M > 12 or K % 8):
        np.testing.assert_array_equal(got, run(op, na.tensor(dev(a)), wt, torch.float32, (M, N)))
    want = oracle.gemm_q4_1(a, blk, N, trans_b=False)
    err = float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), np.sqrt(np.mean(want ** 2))))
    assert err <= 2e-3, err


def test_matmul_q4_1_prepacked_config4_kn():
    """Config 4 with the [K][N/32] weight prepacked: M=1 in full, M=512 on
    sampled rows; at M=512 equal to the raw weight's result bit for bit, at
    M=1 both within the Q4_1 bar of the oracle."""
    import torch
    announce("prepack q4_1 config4")
    K, N = 4096, 14336
    blk = dg.q4_1_blocks(6101, K, N)
    op = na.MatMul(transpose_b=False)
    wt = na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[K, N])
    _, packed = op.prepack(wt)
    for M, rows in ((1, (0, 1)), (512, (300, 316))):
        a = dg.normal(6102 + M, (M, K)).astype(np.float16)
        at = na.tensor(dev(a))
        got_p = run(op, at, packed, torch.float32, (M, N))
        got_r = run(op, at, wt, torch.float32, (M, N))
        if M > 2:
            np.testing.assert_array_equal(got_p, got_r)
        want = oracle.gemm_q4_1(a, blk, N, trans_b=False, rows=rows)
        w = want[rows[0]:rows[1]]
        scale = max(np.max(np.abs(w)), np.sqrt(np.mean(w ** 2)))
        # at M <= 2 the two GEMVs round differently (see above): each within the bar
        for got in (got_p, got_r):
            err = float(np.max(np.abs(got[rows[0]:rows[1]] - w)) / scale)
            assert err <= 2e-3, err


@pytest.mark.parametrize("M", [2, 40])
def test_matmul_q4_1_prepacked_f16_out_and_batched_a(M):
    """f16 A -> f16 C (nnops: the output follows A) through the packed
    planes (the GEMV at M=2, the skinny MFMA GEMM at M=40) and the raw
    weight (the GEMV, the ring), each within the Q4_1 bar; and a batched A
    [2, M, K] against the one packed weight."""
    import torch
    announce(f"prepack q4_1 f16 out / batched M={M}")
    K, N = 1024, 512
    a = dg.normal(900 + M, (2, M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(901 + M, K, N)
    op = na.MatMul(transpose_b=False)
    wt = na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[K, N])
    _, packed = op.prepack(wt)
    at = na.tensor(dev(a))
    got_p = run(op, at, packed, torch.float16, (2, M, N))
    got_r = run(op, at, wt, torch.float16, (2, M, N))
    if M > 2 and not packed_skinny(M, K, True):
        np.testing.assert_array_equal(got_p.view(np.uint16), got_r.view(np.uint16))
    for bi in range(2):
        want = oracle.gemm_q4_1(a[bi], blk, N, trans_b=False, w_round_f16=True, c_f16=True).astype(np.float32)
        scale = max(np.max(np.abs(want)), np.sqrt(np.mean(want ** 2)))
        # at M = 2 the two GEMVs round differently: each within the bar
        for got in (got_p, got_r):
            err = float(np.max(np.abs(got[bi].astype(np.float32) - want)) / scale)
            assert err <= 2e-3, err


@pytest.mark.parametrize("f16_out", [False, True])
@pytest.mark.parametrize("M,K", [(3, 2048), (5, 2048), (8, 2048), (12, 2048), (16, 4096), (33, 1024), (48, 2048),
                                 (5, 1000), (12, 1000)])
def test_matmul_q4_1_prepacked_few_rows(M, K, f16_out):
    """3 <= M <= 48 rows of f16 A over the packed planes: K % 256 == 0 takes
    the skinny MFMA GEMM (weights decoded to f16, one launch per 16 rows:
    within 1e-4 of the oracle with f16-rounded weights), else the one-launch
    GEMV in passes of up to 8 rows (M <= 12; products a * d split exactly).
    Both within the Q4_1 bar of the f32 dequant oracle, every row checked,
    f32 and f16 destinations, N ragged (not a multiple of the 32-column
    block)."""
    import torch
    announce(f"prepack q4_1 few rows M={M} f16_out={f16_out}")
    N = 1000
    a = dg.normal(950 + M, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(951 + M, K, N)
    op = na.MatMul(transpose_b=False)
    wt = na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[K, N])
    _, packed = op.prepack(wt)
    got = run(op, na.tensor(dev(a)), packed, torch.float16 if f16_out else torch.float32, (M, N))
    want = oracle.gemm_q4_1(a, blk, N, trans_b=False)
    if f16_out:
        want = want.astype(np.float16).astype(np.float32)
    scale = max(np.max(np.abs(want)), np.sqrt(np.mean(want ** 2)))
    err = float(np.max(np.abs(got.astype(np.float32) - want)) / scale)
    assert err <= 2e-3, err
    if packed_skinny(M, K, True) and not f16_out:
        assert norm_err(got, oracle.gemm_q4_1(a, blk, N, trans_b=False, w_round_f16=True)) <= 1e-4


@pytest.mark.parametrize("K,N", [(64, 200), (96, 1024), (37, 72)])
def test_q4_1_packed_blob_layout(K, N):
    """The packed q4_1 blob byte for byte, one block column after another:
    the k-blocked nibble plane (block column j: per 8 rows, per nibble dword
    the 8 rows' dwords; rows past K zero), then at align_up(nbn*ceil(K/8)*128,
    256) the d|m plane [nbn][K rounded up to 64] (padding zeroed), restated
    here with numpy from the raw [K][nbn] 20-byte blocks."""
    announce(f"prepack q4_1 blob layout {K}x{N}")
    blk = dg.q4_1_blocks(K * 7 + N, K, N)                # uint8 [K, nbn*20]
    nbn = (N + 31) // 32
    op = na.MatMul(transpose_b=False)
    buf, packed = op.prepack(na.tensor(dev(blk), dtype=na.DT_Q4_1, shape=[K, N]))
    import torch
    torch.cuda.synchronize()
    got = host(buf)
    b3 = blk.reshape(K, nbn, 20)
    kg = (K + 7) // 8
    q32 = np.zeros((kg * 8, nbn, 4), np.uint32)
    q32[:K] = np.ascontiguousarray(b3[:, :, 4:]).view(np.uint32).reshape(K, nbn, 4)
    # [kg][8 rows][nbn][4 dwords] -> [nbn][kg][4 dwords][8 rows]
    nib = q32.reshape(kg, 8, nbn, 4).transpose(2, 0, 3, 1).reshape(-1).view(np.uint8)
    kdm = (K + 63) // 64 * 64
    dm = np.zeros((nbn, kdm, 4), np.uint8)
    dm[:, :K, :] = b3[:, :, :4].transpose(1, 0, 2)
    off = (nbn * kg * 128 + 255) // 256 * 256
    assert na.lib().nnops_hip_prepack_q4_1_bytes(K, N) == off + nbn * kdm * 4
    np.testing.assert_array_equal(got[:nib.size], nib)
    np.testing.assert_array_equal(got[off:off + dm.size], dm.reshape(-1))
