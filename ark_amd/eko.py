"""EKO parameter-buffer sets: tensor order, shapes and per-tensor weight decay.

The order is the one Optimizer::clip_all_grads and Optimizer::step_all walk
(proyecto_ark/ark01/src/optimizer.rs:130-143, :185-227): the tied embedding,
gamma_final, then per layer wq, wk, wv, wo, w1, w2, w3, g1, g2.  Matrices
take the configured weight decay; the RMSNorm gains gamma_final, g1, g2 take
none (optimizer.rs:194-200, :224-226).  Shapes follow memory.rs:227-255
(wq..wo d x d, w1/w3 d x h, w2 h x d, gains d) and the embedding vocab x d.
"""
from dataclasses import dataclass


@dataclass(frozen=True)
class TensorSpec:
    name: str
    shape: tuple
    decay: bool   # takes the configured weight decay
    gain: bool    # RMSNorm gain (initialised to 1.0)

    @property
    def n(self):
        r = 1
        for s in self.shape:
            r *= s
        return r


@dataclass(frozen=True)
class EkoConfig:
    n_layers: int
    d_model: int
    hidden: int
    vocab: int
    n_heads: int = 12

    def tensors(self, with_embedding=True, with_gamma_final=True):
        d, h = self.d_model, self.hidden
        out = []
        if with_embedding:
            out.append(TensorSpec("embed", (self.vocab, d), True, False))
        if with_gamma_final:
            out.append(TensorSpec("gamma_final", (d,), False, True))
        for l in range(self.n_layers):
            out += [
                TensorSpec(f"l{l}.wq", (d, d), True, False),
                TensorSpec(f"l{l}.wk", (d, d), True, False),
                TensorSpec(f"l{l}.wv", (d, d), True, False),
                TensorSpec(f"l{l}.wo", (d, d), True, False),
                TensorSpec(f"l{l}.w1", (d, h), True, False),
                TensorSpec(f"l{l}.w2", (h, d), True, False),
                TensorSpec(f"l{l}.w3", (d, h), True, False),
                TensorSpec(f"l{l}.g1", (d,), False, True),
                TensorSpec(f"l{l}.g2", (d,), False, True),
            ]
        return out

    def n_params(self, **kw):
        return sum(t.n for t in self.tensors(**kw))


# The benchmark configurations:
#   c0: one 768x768 tensor; c1: one EKO layer (9 tensors, no embedding,
#   no gamma_final); c2/c3: EKO-237M (272 tensors); c4: 1.3B scale-up.
EKO_LAYER = EkoConfig(n_layers=1, d_model=768, hidden=2048, vocab=32000)
EKO_237M = EkoConfig(n_layers=30, d_model=768, hidden=2048, vocab=32000)
EKO_1P3B = EkoConfig(n_layers=24, d_model=2048, hidden=5504, vocab=32000, n_heads=16)


SEGMENT = 4096  # ARK_OPT_NORM_SEGMENT: the optimizer cuts every tensor into these


def shard_tensors(specs, rank, world):
    """Rank `rank`'s share of `specs` when `world` GPUs split the optimizer's
    segment list (every tensor cut into SEGMENT-element segments, in table
    order) into contiguous runs of equal length to within one segment: the
    tensors and tensor slices it owns, as 1-D TensorSpecs named
    "name[lo:hi]" for a slice (ZeRO-1 style; w, g, m and v of a slice live
    on its rank)."""
    assert 0 <= rank < world
    counts = [(s.n + SEGMENT - 1) // SEGMENT for s in specs]
    total = sum(counts)
    a, b = rank * total // world, (rank + 1) * total // world
    out, s0 = [], 0
    for spec, c in zip(specs, counts):
        lo, hi = max(a, s0), min(b, s0 + c)
        if lo < hi:
            e0, e1 = (lo - s0) * SEGMENT, min(spec.n, (hi - s0) * SEGMENT)
            if (e0, e1) == (0, spec.n):
                out.append(spec)
            else:
                out.append(TensorSpec(f"{spec.name}[{e0}:{e1}]", (e1 - e0,), spec.decay,
                                      spec.gain))
        s0 += c
    return out


def config_tensors(name):
    """TensorSpec list of a benchmark configuration: c0, c1, c2, c3, c4, or
    c2s8 / c4s8, rank 0's share of c2 / c4 over 8 GPUs (shard_tensors)."""
    if name in ("c2s8", "c4s8"):
        return shard_tensors(config_tensors(name[:2]), 0, 8)
    if name == "c0":
        return [TensorSpec("w", (768, 768), True, False)]
    if name == "c1":
        return EKO_LAYER.tensors(with_embedding=False, with_gamma_final=False)
    if name in ("c2", "c3"):
        return EKO_237M.tensors()
    if name == "c4":
        return EKO_1P3B.tensors()
    raise KeyError(name)
