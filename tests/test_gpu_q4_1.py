"""Q4_1-weight GEMV / GEMM on the GPU through the C ABI (nnops_hip_gemm_q4_1)
against the CPU f32 dequant GEMM oracle (float64 accumulation).

Tolerance (BASELINE: max relative error <= 2e-3 vs the CPU f32 dequant GEMM),
as a normalized relative error: max_i |g_i - w_i| / max(|w_i|, rms(w)), so
outputs that cancel to ~0 do not make the ratio meaningless."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import datagen as dg
import nnops_amd as na
from gpu_util import dev, host, announce, norm_err, oracle_rows, q41_f16_weights

pytestmark = pytest.mark.gpu

TOL = 2e-3


def run_gpu(a, blk, n, *, trans_b, out_f16=False):
    import torch
    M = a.shape[0]
    c = torch.zeros((M, n), dtype=torch.float16 if out_f16 else torch.float32, device="cuda")
    na.gemm_q4_1(dev(a), dev(blk), c, n=n, trans_b=trans_b)
    torch.cuda.synchronize()
    return host(c).astype(np.float32)


CASES = [
    # (M, K, N): GEMV (M <= 2) and MFMA routes; ragged K / N
    (1, 4096, 1024), (2, 4096, 512), (1, 96, 40), (1, 1000, 77), (2, 8200, 64),
    (3, 256, 130), (16, 4096, 256), (64, 512, 300), (130, 1000, 200),
    (1, 4096, 1003), (2, 4096, 77),
    # ring GEMM (K % 64 == 0): ragged M and N tiles, a single k step
    (300, 1024, 520), (7, 64, 256),
    # blocks-along-N ring (row bytes % 16 == 0): ragged M and N, N not a tile multiple
    (300, 1024, 1000), (129, 192, 384), (40, 4096, 2048),
]


@pytest.mark.parametrize("M,K,N", CASES)
@pytest.mark.parametrize("trans_b", [True, False])
def test_q4_1_f16_a_f32_out(M, K, N, trans_b):
    announce(f"q4_1 f16 {M}x{K}x{N} trans_b={trans_b}")
    seed = M * 13 + K + N + int(trans_b)
    a = dg.normal(seed, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(seed + 1, N, K) if trans_b else dg.q4_1_blocks(seed + 2, K, N)
    got = run_gpu(a, blk, N, trans_b=trans_b)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=trans_b)
    err = norm_err(got, want)
    assert err <= TOL, err


@pytest.mark.parametrize("trans_b", [True, False])
def test_q4_1_f32_a(trans_b):
    announce(f"q4_1 f32 A trans_b={trans_b}")
    M, K, N = 5, 640, 96
    a = dg.normal(91, (M, K))
    blk = dg.q4_1_blocks(92, N, K) if trans_b else dg.q4_1_blocks(93, K, N)
    got = run_gpu(a, blk, N, trans_b=trans_b)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=trans_b)
    assert norm_err(got, want) <= 1e-4


@pytest.mark.parametrize("M,K,N", [(3, 4096, 1024), (4, 256, 1000), (8, 512, 64), (16, 4096, 14336), (17, 1024, 520),
                                   (33, 4096, 96), (48, 768, 1030)])
@pytest.mark.parametrize("out_f16", [False, True])
def test_q4_1_skinny(M, K, N, out_f16):
    """3 <= M <= 48 rows of f16 A over [N][K/32] blocks, K % 256 == 0: the
    skinny MFMA kernel (weights decoded to f16, one launch per 16 rows of
    A; ragged N: rows past it are computed and never stored)."""
    import torch
    announce(f"q4_1 skinny {M}x{K}x{N} f16out={out_f16}")
    a = dg.normal(M + K, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(N + 3, N, K)
    got = run_gpu(a, blk, N, trans_b=True, out_f16=out_f16)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=True, w_round_f16=True, c_f16=out_f16).astype(np.float32)
    assert norm_err(got, want) <= TOL


@pytest.mark.parametrize("M,K,N", [(3, 4096, 1024), (16, 512, 1000), (40, 768, 96)])
def test_q4_1_skinny_f32_a(M, K, N):
    """f32 A, 3 <= M <= 48, K % 256 == 0: the skinny kernel's f32 form (f32
    decode, f32 MFMA) against the f64-accumulated oracle within 1e-4."""
    announce(f"q4_1 skinny f32 {M}x{K}x{N}")
    a = dg.normal(M + 2 * K, (M, K))
    blk = dg.q4_1_blocks(N + 5, N, K)
    got = run_gpu(a, blk, N, trans_b=True)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=True)
    assert norm_err(got, want) <= 1e-4


def split_route(M, K, trans_b, N):
    """The f32-A shapes that take a split-f16 ring (gpu_util.q41_f16_weights)."""
    return q41_f16_weights(M, K, False, trans_b, N)


@pytest.mark.parametrize("M,K,N", [(17, 640, 96), (130, 1000, 200), (300, 4096, 520), (16, 96, 40),
                                   (64, 512, 256), (130, 1024, 1000)])
@pytest.mark.parametrize("trans_b", [True, False])
def test_q4_1_f32_a_gemm(M, K, N, trans_b):
    """f32 A past the GEMV rows: the f32 MFMA GEMM (ragged M, N and K tiles)
    against the f64-accumulated oracle within 1e-4 (normalized; an f32 sum of
    K = 4096 products carries ~1e-5); M = 16 is the GEMV loop's last row
    count. The split-f16 rings (K % 64 == 0, either weight form) decode each
    weight to f16 as the f16-A routes do: within 1e-4 of the oracle with the
    weights so rounded (A's two f16 parts carry 22 bits), within BASELINE's
    2e-3 of the exact one."""
    announce(f"q4_1 f32 A GEMM {M}x{K}x{N} trans_b={trans_b}")
    seed = 3 * M + K + N + int(trans_b)
    a = dg.normal(seed, (M, K))
    blk = dg.q4_1_blocks(seed + 1, N, K) if trans_b else dg.q4_1_blocks(seed + 2, K, N)
    got = run_gpu(a, blk, N, trans_b=trans_b)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=trans_b)
    if split_route(M, K, trans_b, N):
        assert norm_err(got, oracle.gemm_q4_1(a, blk, N, trans_b=trans_b, w_round_f16=True)) <= 1e-4
        assert norm_err(got, want) <= TOL
    else:
        assert norm_err(got, want) <= 1e-4


def test_q4_1_f32_a_split_row_scales():
    """The split-f16 ring's per-row power-of-two scaling: rows far outside
    f16's range (1e6 and 1e-7 times N(0,1), one row with a single 1e5 among
    N(0,1), an all-zero row, a row of 2^-130 subnormals) stay within 1e-4 of
    the oracle with f16-rounded weights, row by row."""
    import torch
    M, K, N = 64, 512, 256
    announce(f"q4_1 f32 A split scales {M}x{K}x{N}")
    a = dg.normal(77, (M, K))
    a[0] *= 1e6
    a[1] *= 1e-7
    a[2, 5] = 1e5
    a[3] = 0.0
    a[4] = np.float32(2.0 ** -130) * np.sign(a[4])
    blk = dg.q4_1_blocks(78, N, K)
    assert split_route(M, K, True, N)
    got = run_gpu(a, blk, N, trans_b=True)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=True, w_round_f16=True)
    assert np.all(got[3] == 0.0)
    for m in (0, 1, 2, 4, 5, 63):
        assert norm_err(got[m], want[m]) <= 1e-4, m


@pytest.mark.parametrize("M", [1, 40])
def test_q4_1_f16_out_nnops_semantics(M):
    """f16 A -> f16 C (nnops' dtype rule): the oracle rounds each decoded
    weight to f16 and the output once (test_matmul_q4_1.cpp:203-215)."""
    announce(f"q4_1 f16 out M={M}")
    K, N = 512, 128
    a = dg.normal(95, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(96, N, K)
    got = run_gpu(a, blk, N, trans_b=True, out_f16=True)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=True, w_round_f16=True, c_f16=True).astype(np.float32)
    assert norm_err(got, want) <= TOL


@pytest.mark.parametrize("M", [1, 512])
def test_config4_full(M):
    """BASELINE config 4 at full size: K=4096, N=14336, f16 A ~ N(0,1), f32 out;
    every output checked (the oracle in row bands over the host's cores)."""
    announce(f"config4 M={M}")
    K, N = 4096, 14336
    a = dg.normal(100 + M, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(101, N, K)
    got = run_gpu(a, blk, N, trans_b=True)
    want = oracle_rows(lambda r0, r1: oracle.gemm_q4_1(a, blk, N, trans_b=True, rows=(r0, r1))[r0:r1], M, band=4)
    err = norm_err(got, want)
    assert err <= TOL, err


def test_config4_kn_m512():
    """Config 4 with the [K][N/32] weight layout (blocks along N), M=512,
    every output checked."""
    announce("config4 kn M=512")
    M, K, N = 512, 4096, 14336
    a = dg.normal(612, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(613, K, N)
    got = run_gpu(a, blk, N, trans_b=False)
    want = oracle_rows(lambda r0, r1: oracle.gemm_q4_1(a, blk, N, trans_b=False, rows=(r0, r1))[r0:r1], M, band=4)
    err = norm_err(got, want)
    assert err <= TOL, err


@pytest.mark.parametrize("M", [1, 2])
def test_config4_kn_gemv_full(M):
    """Config 4's literal [K][N/32] weight at M = 1 and 2, every output
    checked: the one-launch GEMV whose K splits meet in the last-arriving
    workgroup of each column group."""
    announce(f"config4 kn gemv M={M}")
    K, N = 4096, 14336
    a = dg.normal(700 + M, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(702, K, N)
    got = run_gpu(a, blk, N, trans_b=False)
    want = oracle.gemm_q4_1(a, blk, N, trans_b=False)
    err = norm_err(got, want)
    print(f"config4 kn gemv M={M}: normalized error {err:.3e}")
    assert err <= TOL, err


@pytest.mark.parametrize("M,K,N", [(1, 2048, 3000), (2, 96, 1056), (1, 4160, 512)])
def test_kn_gemv_padded_rows_and_repeat(M, K, N):
    """Blocks along N with a padded row pitch (16-byte multiple, wider than the
    blocks) and a last, narrower column group; a second call on the same
    workspace (counters left by the first) gives the same bits."""
    import torch
    announce(f"q4_1 kn padded {M}x{K}x{N}")
    a = dg.normal(710 + K, (M, K)).astype(np.float16)
    blk = dg.q4_1_blocks(711 + N, K, N)
    row = blk.shape[1]
    pitch = (row + 16 + 15) // 16 * 16
    padded = np.full((K, pitch), 0xA5, dtype=np.uint8)
    padded[:, :row] = blk
    bp = dev(padded)
    ad = dev(a)
    ws = torch.empty(8 << 20, dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(2):
        c = torch.zeros((M, N), dtype=torch.float32, device="cuda")
        na.gemm_q4_1(ad, bp, c, n=N, trans_b=False, ldb_bytes=pitch, workspace=ws)
        torch.cuda.synchronize()
        outs.append(host(c))
    want = oracle.gemm_q4_1(a, blk, N, trans_b=False)
    assert norm_err(outs[0].astype(np.float32), want) <= TOL
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
