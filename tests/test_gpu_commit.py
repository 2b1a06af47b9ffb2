"""GPU Poseidon Merkle commitments (gkr_weight_commitment, gkr_weight_commitments,
gkr_mle_commitment) against the reference's SP3 weight commitment and the CPU oracle; at
full Qwen shapes, against the padding identity (a matrix padded with explicit zero rows and
columns to the power-of-two grid commits to the same root, since the grid's padding cells are
SecureField zero)."""
import numpy as np
import oracle as O
import pytest

P = (1 << 31) - 1
pytestmark = pytest.mark.gpu


def rand_matrix(rng, r, c):
    return rng.integers(0, P, size=(r, c), dtype=np.uint32)


def test_sp3_weight_commitment(gpu_ctx, golden):
    B = np.array([[2 * i + j + 1 for j in range(2)] for i in range(4)], dtype=np.uint32)
    m = gpu_ctx.upload(B)
    assert gpu_ctx.weight_commitment(m) == int(golden["sp3"]["weight_commitments"][0], 16)


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 2), (2, 1), (1, 7), (7, 1), (3, 5), (4, 4), (16, 16), (17, 33),
                                       (100, 7), (33, 200), (256, 64), (5, 1000)])
def test_weight_commitment_matches_oracle(gpu_ctx, rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    B = rand_matrix(rng, rows, cols)
    print(f"weight commitment {rows}x{cols}", flush=True)
    assert gpu_ctx.weight_commitment(gpu_ctx.upload(B)) == O.weight_commitment(B)


def test_weight_commitment_edge_values(gpu_ctx):
    for v in (0, 1, P - 1):
        B = np.full((3, 6), v, dtype=np.uint32)
        assert gpu_ctx.weight_commitment(gpu_ctx.upload(B)) == O.weight_commitment(B)


def test_batch_equals_single(gpu_ctx):
    rng = np.random.default_rng(9)
    shapes = [(4, 2), (1, 1), (64, 48), (5, 300), (130, 3), (1, 1024), (256, 256)]
    mats = [rand_matrix(rng, r, c) for r, c in shapes]
    dev = [gpu_ctx.upload(B) for B in mats]
    roots = gpu_ctx.weight_commitments(dev)
    assert roots == [gpu_ctx.weight_commitment(m) for m in dev]
    assert roots[0] == O.weight_commitment(mats[0]) and roots[2] == O.weight_commitment(mats[2])
    assert gpu_ctx.weight_commitments([]) == []


@pytest.mark.parametrize("n", [1, 2, 3, 5, 16, 1000, 4096])
def test_mle_commitment_matches_oracle(gpu_ctx, n):
    rng = np.random.default_rng(n)
    q = rng.integers(0, P, size=(n, 4), dtype=np.uint32)
    print(f"mle commitment n={n}", flush=True)
    assert gpu_ctx.mle_commitment(gpu_ctx.qvec_upload(q)) == O.mle_commitment(q)


@pytest.mark.parametrize("rows,cols", [(300, 200), (5120, 1024), (5120, 5120), (13824, 5120)])
def test_explicit_zero_padding_gives_same_root(gpu_ctx, rows, cols):
    """B and B padded with explicit zeros to next_pow2(rows) x next_pow2(cols) commit alike:
    the padded run hashes every grid cell through the leaf path, the plain run takes the
    padding subtrees from the table."""
    pk, pn = 1 << (rows - 1).bit_length(), 1 << (cols - 1).bit_length()
    print(f"padding identity {rows}x{cols} -> {pk}x{pn}", flush=True)
    a = gpu_ctx.synthetic(rows, cols, 0, rows + cols)
    B = a.download()
    Bp = np.zeros((pk, pn), dtype=np.uint32)
    Bp[:rows, :cols] = B
    b = gpu_ctx.upload(Bp)
    ra, rb = gpu_ctx.weight_commitments([a, b])
    assert ra == rb
    # a changed entry changes the root
    B[rows // 2, cols // 3] = (int(B[rows // 2, cols // 3]) + 1) % P
    assert gpu_ctx.weight_commitment(gpu_ctx.upload(B)) != ra


def test_commitment_cache(gpu_ctx):
    """The weight-commitment cache on resident matrices (the reference's WeightCommitmentCache,
    weight_cache.rs:283-327): a computed root is kept on its matrix and returned again, a batch mixing
    cached and uncached weights equals the uncached batch, a root seeded with set_commitment is
    used as given, and invalidate / forward_into drop it."""
    print("case commitment cache", flush=True)
    rng = np.random.default_rng(21)
    Bs = [rand_matrix(rng, 33, 20), rand_matrix(rng, 64, 64), rand_matrix(rng, 7, 300)]
    ms = [gpu_ctx.upload(B) for B in Bs]
    want = [O.weight_commitment(B) for B in Bs]
    assert all(m.cached_commitment() is None for m in ms)
    assert gpu_ctx.weight_commitment(ms[1]) == want[1]
    assert ms[1].cached_commitment() == want[1] and ms[0].cached_commitment() is None
    assert gpu_ctx.weight_commitments(ms) == want  # one cached, two computed
    assert [m.cached_commitment() for m in ms] == want
    assert gpu_ctx.weight_commitments(ms) == want  # all cached
    # a root persisted elsewhere and seeded on a new handle of the same weight
    again = gpu_ctx.upload(Bs[2])
    again.set_commitment(want[2])
    assert again.cached_commitment() == want[2] and gpu_ctx.weight_commitment(again) == want[2]
    # the contents change: the root is dropped and the new one computed
    ms[0].invalidate()
    assert ms[0].cached_commitment() is None
    assert gpu_ctx.weight_commitment(ms[0]) == want[0]
    ident = gpu_ctx.upload(np.eye(64, dtype=np.uint32))
    B2 = rand_matrix(rng, 64, 64)
    gpu_ctx.matmul_forward_into(ident, gpu_ctx.upload(B2), ms[1])
    assert ms[1].cached_commitment() is None
    assert gpu_ctx.weight_commitment(ms[1]) == O.weight_commitment(B2)
