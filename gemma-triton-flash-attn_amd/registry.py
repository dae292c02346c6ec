"""HEAD_DIM-keyed kernel-config registry.

The reference keeps its tile choices as if/else tables keyed on HEAD_DIM inside the
launch code (/root/reference/flash_attn/attention.py:561-579 inference forward,
1445-1451 training forward, 1498-1504 dQ, 1536-1564 dKV, 1576-1587 Q_SPLITS). Here the
same role is one explicit table. Each entry names the tiles of the three gfx950 kernels:
the forward runs one wave per 32 query rows over the full head dim, the dQ kernel
``dq_split`` waves per 32 query rows (a pair splitting the head dim at D=512, one wave at
D <= 256), the dK/dV kernel ``dkv_roles`` waves per 32 keys (a role-split pair at D=512 and
D=128, one wave doing all four products at D=256 and D=64; with a sliding window D=256 runs
role-split pairs at two waves per SIMD, the ``dkv_window`` form). D=64 and D=128 cover the rest
of the reference's documented head-dim range (64-512, powers of two; docs/api.md:63).

The C library holds the same table (csrc/gfa_api.hip, kRegistry); ``gfa_config`` reports
what the library will use and the tests assert the two agree.
"""
from __future__ import annotations

from dataclasses import dataclass

NUM_CUS = 256  # MI355X compute units; the Q-split target is one workgroup per CU


@dataclass(frozen=True)
class KernelConfig:
    head_dim: int
    fwd_block_kv: int   # keys per LDS tile in the forward
    fwd_waves: int      # waves per forward workgroup (pairs = waves / 2)
    dq_block_kv: int
    dq_waves: int
    dq_split: int       # waves per 32 query rows in the dQ kernel (2: head-dim halves; 1: full)
    dkv_block_q: int    # queries per LDS tile in the dKV kernel
    dkv_waves: int
    dkv_roles: int      # waves per 32 keys in the dKV kernel (2: role-split pair; 1: one wave)
    dkv_wgs_per_cu: int = 1  # dKV workgroups resident per CU (waves per SIMD)
    fwd_block_kv_options: tuple = ()  # other built forward tile widths (BLOCK_KV override)
    fwd_block_kv_window: int = 0      # forward tile with a sliding window (0 = fwd_block_kv)
    # dK/dV form with a sliding window shorter than the sequence, (waves, roles, wgs_per_cu);
    # () = the same as without one
    dkv_window: tuple = ()

    def dkv_form(self, windowed: bool) -> tuple:
        """(waves, roles, workgroups per CU) of the dK/dV kernel."""
        if windowed and self.dkv_window:
            return self.dkv_window
        return (self.dkv_waves, self.dkv_roles, self.dkv_wgs_per_cu)


REGISTRY: dict[int, KernelConfig] = {
    512: KernelConfig(512, fwd_block_kv=32, fwd_waves=4, dq_block_kv=32, dq_waves=4, dq_split=2, dkv_block_q=32,
                      dkv_waves=4, dkv_roles=2,
                      fwd_block_kv_options=(32,)),
    256: KernelConfig(256, fwd_block_kv=32, fwd_waves=4, dq_block_kv=32, dq_waves=4, dq_split=1, dkv_block_q=32,
                      dkv_waves=4, dkv_roles=1, dkv_window=(4, 2, 2),
                      fwd_block_kv_options=(32, 64)),
    128: KernelConfig(128, fwd_block_kv=64, fwd_waves=4, dq_block_kv=32, dq_waves=4, dq_split=1, dkv_block_q=32,
                      dkv_waves=4, dkv_roles=2,
                      dkv_wgs_per_cu=2, fwd_block_kv_options=(32, 64), fwd_block_kv_window=32),
    64: KernelConfig(64, fwd_block_kv=64, fwd_waves=4, dq_block_kv=32, dq_waves=4, dq_split=1, dkv_block_q=32,
                     dkv_waves=4, dkv_roles=1, dkv_wgs_per_cu=2,
                     fwd_block_kv_options=(32, 64)),
}

SUPPORTED_HEAD_DIMS = tuple(sorted(REGISTRY))


def lookup(head_dim: int) -> KernelConfig:
    try:
        return REGISTRY[head_dim]
    except KeyError:
        raise ValueError(f"head_dim={head_dim} is not in the registry {SUPPORTED_HEAD_DIMS}") from None


def _pow2_divisor_le(r: int, cap: int) -> int:
    x = 1
    while x * 2 <= cap and r % (x * 2) == 0:
        x *= 2
    return x


def query_grid(batch: int, heads_q: int, heads_kv: int, seq_len: int, units: int) -> dict:
    """Workgroup decomposition of the forward / dQ kernels (pack-GQA).

    A workgroup holds ``units`` 32-row query blocks (one per wave in the forward kernel,
    one per wave pair in the dQ kernel): ``hpw`` query heads of one KV head times ``qbw``
    neighbouring 32-row blocks.
    """
    r = heads_q // heads_kv
    hpw = _pow2_divisor_le(r, units)
    qbw = units // hpw
    n_qsb = -(-seq_len // (32 * qbw))
    return {"hpw": hpw, "qbw": qbw, "block_q": 32 * qbw, "n_hg": r // hpw, "n_qsb": n_qsb,
            "nblocks": n_qsb * batch * heads_kv * (r // hpw)}


def q_splits_for(batch: int, heads_kv: int, seq_len: int, units: int, wgs_per_cu: int = 1,
                 full_causal: bool = True) -> int:
    """Smallest of {1, 2, 4, 8} that fills the GPU with dKV workgroups (``units`` = 32-key
    units per workgroup, ``wgs_per_cu`` = workgroups resident per CU).

    Same intent as the reference's Q_SPLITS rule (attention.py:1576-1587): split each key
    block's query range only when the raw grid is small. A full-causal grid asks for two
    rounds of NUM_CUS * wgs_per_cu workgroups (its key blocks carry unequal work, which the
    kernel's heaviest-first grid order balances once there are two rounds); windowed and
    non-causal grids have near-uniform work and ask for one. Measured on MI355X on grids of
    32 to 1024 workgroups at D = 64..512; beyond that a split only adds fp32 partial traffic.
    """
    keys_per_wg = 32 * units
    grid = -(-seq_len // keys_per_wg) * batch * heads_kv
    want = (2 if full_causal else 1) * NUM_CUS * wgs_per_cu
    qs = 1
    while qs < 8 and grid * qs < want:
        qs *= 2
    return qs


def q_splits_for_problem(batch: int, heads_kv: int, seq_len: int, head_dim: int, causal: bool = True,
                         window: int = 0) -> int:
    """The split count gfa_bwd uses (q_splits = 0) for one problem."""
    c = lookup(head_dim)
    windowed = causal and 0 < window < seq_len
    waves, roles, wgs = c.dkv_form(windowed)
    return q_splits_for(batch, heads_kv, seq_len, waves // roles, wgs, causal and not windowed)


def get_config(batch: int, heads_q: int, heads_kv: int, seq_len: int, head_dim: int) -> dict:
    """Everything the library decides for one problem (same keys as ``gfa_config``)."""
    c = lookup(head_dim)
    fq = query_grid(batch, heads_q, heads_kv, seq_len, c.fwd_waves)
    dq = query_grid(batch, heads_q, heads_kv, seq_len, c.dq_waves // c.dq_split)
    return {
        "head_dim": head_dim,
        "fwd_block_q": fq["block_q"],
        "fwd_block_kv": c.fwd_block_kv,
        "fwd_waves": c.fwd_waves,
        "dq_block_q": dq["block_q"],
        "dq_block_kv": c.dq_block_kv,
        "dq_waves": c.dq_waves,
        "dkv_block_kv": 32 * (c.dkv_waves // c.dkv_roles),
        "dkv_block_q": c.dkv_block_q,
        "dkv_waves": c.dkv_waves,
        "q_splits": q_splits_for_problem(batch, heads_kv, seq_len, head_dim, True, 0),
    }
