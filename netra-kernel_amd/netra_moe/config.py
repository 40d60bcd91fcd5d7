"""Shapes of the routed-MoE layer and the derived buffer sizes.

The layer contract follows the reference's MoE engine manifest
(manifests/gfx950/models/qwen36-35b-c64-fp8.json:6-13, 43-49): hidden H,
intermediate I, E routed experts plus S always-on shared experts stored as
expert ids E..E+S-1, top-K routed slots plus the shared slot, FP8 E4M3 weights
with 128x128 fp32 block scales and 1x128 activation scales, 64-row sorted
expert blocks with capacity ceil(routes / 64) + experts blocks.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, field

BLOCK_M = 64          # rows per sorted expert block (reference NETRA_ROUTE_BLOCK)
SCALE_BLOCK = 128     # quantisation block edge


@dataclass(frozen=True)
class MoEConfig:
    name: str
    T: int            # tokens in one layer call
    H: int            # hidden size
    E: int            # routed experts
    K: int            # routed top-k
    I: int            # expert intermediate size
    S: int = 0        # shared experts (0 or 1)
    router_bias: str = "none"   # "none" | "zipf1.1": log-Zipf(1.1) expert bias | "hot": +64 on experts 0..K-1
    seed: int = 0
    notes: str = field(default="", compare=False)

    def __post_init__(self) -> None:
        if self.T < 1 or self.T >= (1 << 24):
            raise ValueError("T must be in [1, 2^24)")
        if self.H % SCALE_BLOCK or self.I % SCALE_BLOCK or self.H <= 0 or self.I <= 0:
            raise ValueError("H and I must be positive multiples of 128")
        if self.H % 256:
            raise ValueError("H must be a multiple of 256 (down-GEMM column groups)")
        if not 1 <= self.K <= self.E or self.K > 63:
            raise ValueError("need 1 <= K <= min(E, 63)")
        if self.S not in (0, 1):
            raise ValueError("S must be 0 or 1")
        if self.E > 512:
            raise ValueError("E must be <= 512")
        if self.router_bias not in ("none", "zipf1.1", "hot"):
            raise ValueError("unknown router_bias")

    # ---- derived sizes ------------------------------------------------------
    @property
    def Ktot(self) -> int:
        return self.K + self.S

    @property
    def Etot(self) -> int:
        return self.E + self.S

    @property
    def router_rows(self) -> int:
        return self.E + self.S

    @property
    def routes(self) -> int:
        return self.T * self.Ktot

    @property
    def mask_words_per_expert(self) -> int:
        return (self.T + 63) // 64

    @property
    def cap_blocks(self) -> int:
        return (self.routes + BLOCK_M - 1) // BLOCK_M + self.Etot

    @property
    def cap_rows(self) -> int:
        return self.cap_blocks * BLOCK_M

    @property
    def sort_lds_bytes(self) -> int:
        """Dynamic LDS of the sort kernel (sort_base_words / sort_mask_in_lds
        in moe_router.hip): prefix, block / tile / pair offsets, wave totals and
        block owners, plus
        a copy of the routing bitmask when the total stays within 160 KiB."""
        ew = self.Etot * self.mask_words_per_expert
        base = (ew + 4 * self.Etot + 3 + 48 + self.cap_blocks + 1) & ~1
        with_mask = 4 * (base + 2 * ew)
        return with_mask if with_mask <= 160 * 1024 else 4 * base

    @property
    def cap_tiles(self) -> int:
        """Upper bound on non-empty 16-row tiles: sum over experts of ceil(rows / 16)."""
        return (self.routes + 15) // 16 + self.Etot

    def flops(self) -> int:
        """Algorithmic FLOPs of one layer call: router + every routed/shared row."""
        return 2 * self.T * self.H * self.router_rows + self.routes * (2 * self.H * 2 * self.I + 2 * self.I * self.H)

    def expert_bytes(self) -> int:
        """HBM bytes of one expert's FP8 weights plus fp32 block scales."""
        w = 2 * self.I * self.H + self.H * self.I
        s = 4 * ((2 * self.I // 128) * (self.H // 128) + (self.H // 128) * (self.I // 128))
        return w + s

    def algorithmic_bytes(self, touched_experts: int) -> int:
        """Bytes a perfect single pass moves: touched experts' weights + router
        weights + bias + x in + out."""
        return (touched_experts * self.expert_bytes() + 2 * self.H * self.router_rows
                + 4 * self.E + 2 * self.T * self.H + 2 * self.T * self.H)

    def to_dict(self) -> dict:
        d = asdict(self)
        d.update(Ktot=self.Ktot, Etot=self.Etot, cap_blocks=self.cap_blocks)
        return d


# BASELINE.json configs[0..4]
BASELINE_CONFIGS: dict[str, MoEConfig] = {
    "cpu_small": MoEConfig("cpu_small", T=16, H=512, E=16, K=2, I=256, S=0, seed=1000),
    "decode_t64": MoEConfig("decode_t64", T=64, H=2048, E=256, K=8, I=512, S=1, seed=1001),
    "decode_t1": MoEConfig("decode_t1", T=1, H=2048, E=256, K=8, I=512, S=1, seed=1002),
    "verify_t512": MoEConfig("verify_t512", T=512, H=2048, E=256, K=8, I=512, S=1,
                             router_bias="zipf1.1", seed=1003,
                             notes="64 requests x 8 draft tokens"),
    "prefill_t4096": MoEConfig("prefill_t4096", T=4096, H=2048, E=256, K=8, I=512, S=1, seed=1004),
}
