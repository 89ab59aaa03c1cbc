"""A synthetic corpus for the sweep protocol when no SuiteSparse files are at hand: 24 seeded
matrices of the structure classes such corpora hold (uniform random, power-law graphs, bands, 2D
and 3D stencils, block-sparse, R-MAT, arrow), written as Matrix Market files with the corpus CSV
the sweep reads (group,name,rows,cols,nnz; the columns of bench200/corpus200.csv).

    python -m vcsr_mc_amd.synth_corpus OUTDIR [--scale S]
    python -m vcsr_mc_amd.sweep all --corpus OUTDIR/corpus.csv --mtx-dir OUTDIR/mtx --O 128

--scale multiplies every size (1.0: 0.1-2.4 M nonzeros per matrix)."""
import argparse
import os

import numpy as np

SEED = 20261201


class Corpus:
    def __init__(self, out: str, scale: float = 1.0):
        self.out, self.scale = out, scale
        self.rng = np.random.default_rng(SEED)
        self.rows = ["group,name,rows,cols,nnz"]
        os.makedirs(os.path.join(out, "mtx"), exist_ok=True)

    def n(self, x: int, lo: int = 4) -> int:
        return max(lo, int(round(x * self.scale)))

    def write(self, name, group, M, N, r, c):
        """Distinct (r, c) entries in row-major order, values U[-1, 1]."""
        key = np.unique(np.asarray(r, np.int64) * N + np.asarray(c, np.int64))
        r, c = key // N, key % N
        v = self.rng.uniform(-1, 1, r.size)
        with open(os.path.join(self.out, "mtx", name + ".mtx"), "w") as fh:
            fh.write(f"%%MatrixMarket matrix coordinate real general\n{M} {N} {r.size}\n")
            np.savetxt(fh, np.column_stack([r + 1, c + 1, v]), fmt=["%d", "%d", "%.6f"])
        self.rows.append(f"{group},{name},{M},{N},{r.size}")

    def uniform(self, name, M, N, k):
        M, N = self.n(M), self.n(N)
        r = np.repeat(np.arange(M), self.rng.poisson(k, M))
        self.write(name, "random", M, N, r, self.rng.integers(0, N, r.size))

    def power_law(self, name, N, alpha, avg):
        """Configuration model: Zipf(alpha) degrees scaled to the mean, stubs paired at random,
        both directions kept (symmetric pattern)."""
        N = self.n(N, 8)
        d = np.minimum(self.rng.zipf(alpha, N), N // 4).astype(np.float64)
        d = np.maximum(1, np.round(d * avg * N / d.sum())).astype(np.int64)
        stubs = np.repeat(np.arange(N), d)
        self.rng.shuffle(stubs)
        h = stubs.size // 2
        a, b = stubs[:h], stubs[h:2 * h]
        self.write(name, "powerlaw", N, N, np.concatenate([a, b]), np.concatenate([b, a]))

    def band(self, name, N, bw):
        N = self.n(N)
        r = np.repeat(np.arange(N), 2 * bw + 1)
        c = r + np.tile(np.arange(-bw, bw + 1), N)
        keep = (c >= 0) & (c < N)
        self.write(name, "banded", N, N, r[keep], c[keep])

    def stencil(self, name, n, dims, full):
        """Natural-order grid of side n in 2 or 3 dimensions; 5/7-point or 9/27-point."""
        n = max(3, int(round(n * self.scale ** (1.0 / dims))))
        idx = np.indices((n,) * dims).reshape(dims, -1)
        v = np.ravel_multi_index(idx, (n,) * dims)
        rr, cc = [], []
        for off in np.ndindex((3,) * dims):
            o = np.array(off) - 1
            if not full and np.abs(o).sum() > 1:
                continue
            nb = idx + o[:, None]
            ok = np.all((nb >= 0) & (nb < n), axis=0)
            rr.append(v[ok])
            cc.append(np.ravel_multi_index(nb[:, ok], (n,) * dims))
        self.write(name, "stencil", n ** dims, n ** dims, np.concatenate(rr), np.concatenate(cc))

    def block(self, name, nb, bs, per):
        """nb block rows of height bs, each with `per` dense bs x bs blocks at random block
        columns."""
        nb = self.n(nb)
        br = np.repeat(np.arange(nb), per)
        bc = self.rng.integers(0, nb, br.size)
        ii, jj = np.meshgrid(np.arange(bs), np.arange(bs), indexing="ij")
        r = (br[:, None] * bs + ii.ravel()[None, :]).ravel()
        c = (bc[:, None] * bs + jj.ravel()[None, :]).ravel()
        self.write(name, "block", nb * bs, nb * bs, r, c)

    def rmat(self, name, scale, edge_factor):
        """R-MAT with (a, b, c, d) = (0.57, 0.19, 0.19, 0.05), duplicates merged."""
        scale = max(4, scale + int(np.floor(np.log2(max(self.scale, 1e-9)))))
        n = 1 << scale
        m = edge_factor * n
        r = np.zeros(m, np.int64)
        c = np.zeros(m, np.int64)
        for bit in range(scale):
            q = np.searchsorted([0.57, 0.76, 0.95], self.rng.random(m), side="right")
            r |= (q >> 1).astype(np.int64) << bit
            c |= (q & 1).astype(np.int64) << bit
        self.write(name, "rmat", n, n, r, c)

    def arrow(self, name, N, w):
        """Diagonal plus w dense rows and w dense columns."""
        N = self.n(N)
        r = np.concatenate([np.arange(N), np.repeat(np.arange(w), N), np.tile(np.arange(N), w)])
        c = np.concatenate([np.arange(N), np.tile(np.arange(N), w), np.repeat(np.arange(w), N)])
        self.write(name, "arrow", N, N, r, c)

    def finish(self):
        with open(os.path.join(self.out, "corpus.csv"), "w") as fh:
            fh.write("\n".join(self.rows) + "\n")


def make(out: str, scale: float = 1.0) -> str:
    k = Corpus(out, scale)
    k.uniform("rand_20k_8", 20000, 20000, 8)
    k.uniform("rand_100k_16", 100000, 100000, 16)
    k.uniform("rand_50k_32", 50000, 50000, 32)
    k.uniform("rand_rect_20k_100k", 20000, 100000, 20)
    k.uniform("rand_2k_50", 2000, 2000, 50)
    k.power_law("plaw_50k_a21", 50000, 2.1, 10)
    k.power_law("plaw_200k_a25", 200000, 2.5, 6)
    k.power_law("plaw_100k_a18", 100000, 1.8, 12)
    k.band("band_100k_3", 100000, 3)
    k.band("band_50k_16", 50000, 16)
    k.stencil("grid2d_500_5pt", 500, 2, False)
    k.stencil("grid2d_300_9pt", 300, 2, True)
    k.stencil("grid3d_60_7pt", 60, 3, False)
    k.stencil("grid3d_40_27pt", 40, 3, True)
    k.block("block_b8_4k", 4096, 8, 6)
    k.block("block_b16_2k", 2048, 16, 4)
    k.block("block_b32_1k", 1024, 32, 4)
    k.block("block_b4_20k", 20000, 4, 5)
    k.rmat("rmat_16", 16, 16)
    k.rmat("rmat_17", 17, 8)
    k.arrow("arrow_100k_4", 100000, 4)
    k.uniform("rand_300k_3", 300000, 300000, 3)
    k.stencil("grid2d_700_5pt", 700, 2, False)
    k.power_law("plaw_30k_a30", 30000, 3.0, 20)
    k.finish()
    return os.path.join(out, "corpus.csv")


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("out")
    p.add_argument("--scale", type=float, default=1.0)
    a = p.parse_args(argv)
    print(make(a.out, a.scale))


if __name__ == "__main__":
    main()
