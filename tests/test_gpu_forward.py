"""Forward-pass matrix product on the matrix cores (gkr_matmul_forward) against the oracle's
exact M31 product, and at Qwen shapes through the prover's own output claim (MLE of A.B at a
random point, computed from the restrictions, never from C)."""
import gkr_mi355x as G
import numpy as np
import oracle as O
import pytest

pytestmark = pytest.mark.gpu
P = (1 << 31) - 1


def lg(v):
    return max(0, (v - 1).bit_length())


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (1, 4, 2), (3, 5, 7), (2, 31, 33), (1, 64, 300), (33, 100, 70),
                                   (64, 300, 257), (65, 129, 65), (130, 40, 3), (7, 1000, 9)])
def test_forward_matches_oracle(gpu_ctx, m, k, n):
    print(f"forward {m}x{k} . {k}x{n}", flush=True)
    rng = np.random.default_rng(m * 10007 + k * 101 + n)
    A = rng.integers(0, P, size=(m, k), dtype=np.uint32)
    B = rng.integers(0, P, size=(k, n), dtype=np.uint32)
    C = gpu_ctx.matmul_forward(gpu_ctx.upload(A), gpu_ctx.upload(B)).download()
    assert np.array_equal(C, O.matmul_forward(A, B))


def test_forward_edge_values_and_int8_range(gpu_ctx):
    rng = np.random.default_rng(3)
    for fill in (P - 1, 0, 1, P // 2, P // 2 + 1):
        A = np.full((5, 77), fill, dtype=np.uint32)
        B = np.full((77, 6), P - 1, dtype=np.uint32)
        assert np.array_equal(gpu_ctx.matmul_forward(gpu_ctx.upload(A), gpu_ctx.upload(B)).download(),
                              O.matmul_forward(A, B))
    # int8-range values (negatives as P - |x|), as the configs' weights and activations
    A = O.synthetic(64, 576, 1, 5)
    B = O.synthetic(576, 192, 1, 6)
    assert np.array_equal(gpu_ctx.matmul_forward(gpu_ctx.upload(A), gpu_ctx.upload(B)).download(),
                          O.matmul_forward(A, B))


def test_forward_long_k_splits(gpu_ctx):
    """K above one split's 16384 limit and not a multiple of 32."""
    rng = np.random.default_rng(8)
    A = rng.integers(0, P, size=(2, 40001), dtype=np.uint32)
    B = rng.integers(0, P, size=(40001, 3), dtype=np.uint32)
    assert np.array_equal(gpu_ctx.matmul_forward(gpu_ctx.upload(A), gpu_ctx.upload(B)).download(),
                          O.matmul_forward(A, B))


def test_forward_shape_errors(gpu_ctx):
    a = gpu_ctx.upload(np.ones((2, 3), dtype=np.uint32))
    with pytest.raises(G.GkrError):
        gpu_ctx.matmul_forward(a, gpu_ctx.upload(np.ones((4, 2), dtype=np.uint32)))


@pytest.mark.parametrize("name,m,k,n", [("q", 64, 5120, 5120), ("k", 64, 5120, 1024), ("gate", 64, 5120, 13824),
                                        ("down", 64, 13824, 5120)])
def test_forward_qwen_shapes_by_claim(gpu_ctx, name, m, k, n):
    """MLE of the GPU product at a random point equals the prover's output claim
    (sum f_a * f_b of the restrictions of A and B), for int8-range and uniform M31 data."""
    for kind in (1, 0):
        print(f"forward qwen {name} kind {kind}", flush=True)
        a = gpu_ctx.synthetic(m, k, kind, 21)
        b = gpu_ctx.synthetic(k, n, kind, 22)
        c = gpu_ctx.matmul_forward(a, b)
        ch = G.PoseidonChannel()
        ch.mix_u64(k + kind)
        r = ch.draw_qm31s(lg(m) + lg(n))
        claim = gpu_ctx.matmul_output_claim(a, b, r)
        C = c.download()
        pm, pn = 1 << lg(m), 1 << lg(n)
        mle = np.zeros((pm, pn, 4), dtype=np.uint32)
        mle[:m, :n, 0] = C
        got = gpu_ctx.evaluate_mle_at_point([tuple(v) for v in mle.reshape(-1, 4)], r)
        assert got == claim


def test_forward_into_and_variants(gpu_ctx):
    """gkr_matmul_forward_into over a reused output; int8-range A with a full-range B and the
    reverse (the 1- and 4-plane kernels on either side)."""
    rng = np.random.default_rng(12)
    for kinds in ((1, 0), (0, 1), (1, 1), (0, 0)):
        A = O.synthetic(40, 300, kinds[0], 7)
        B = O.synthetic(300, 50, kinds[1], 8)
        a, b = gpu_ctx.upload(A), gpu_ctx.upload(B)
        out = gpu_ctx.matmul_forward(a, b)
        assert np.array_equal(out.download(), O.matmul_forward(A, B))
        A2 = rng.integers(0, P, size=(40, 300), dtype=np.uint32) if kinds[0] == 0 else O.synthetic(40, 300, 1, 9)
        gpu_ctx.matmul_forward_into(gpu_ctx.upload(A2), b, out)
        assert np.array_equal(out.download(), O.matmul_forward(A2, B))
    with pytest.raises(G.GkrError):
        gpu_ctx.matmul_forward_into(a, b, a)
