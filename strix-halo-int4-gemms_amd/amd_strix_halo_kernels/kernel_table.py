"""Python mirror of the gfx950 kernel table compiled into the library.

The library (csrc/k_dense.hip, csrc/k_ragged.hip) appends its kernels in a
fixed order; this module lists the same entries in the same order so that the
registry can be built without loading the library.  ``native`` checks the
mirror against ``amd_strix_halo_kernels_kernel_table_entry`` the first time it
loads the library and refuses to launch on a mismatch.

This table replaces the reference's tuned gfx1151 tile seeds
(registry.py:112-176) and per-kernel JSON launch metadata.
"""

from __future__ import annotations

import functools
from dataclasses import dataclass

FAMILY_DENSE = 0
FAMILY_RAGGED_FWD = 1
FAMILY_RAGGED_BWD = 2

LAYOUT_NN = 0
LAYOUT_NT = 1
LAYOUT_TN = 2
LAYOUT_TT = 3
LAYOUT_CODES = {"nn": LAYOUT_NN, "nt": LAYOUT_NT, "tn": LAYOUT_TN, "tt": LAYOUT_TT}

SCALE_PER_CHANNEL = 0
SCALE_SUBCHANNEL = 1

EPI_KIND_PLAIN = 0
EPI_KIND_SWIGLU = 2

EPILOGUE_NONE = 0
EPILOGUE_RELU2 = 1
EPILOGUE_SWIGLU = 2

OUT_BF16 = 0
OUT_F32 = 1
OUT_I32 = 2

# Operand formats: PACKED entries read A and B as given; FP6 entries convert
# both int4 operands into a caller workspace in the fp6 (e2m3, v/8) block format
# first (amd_strix_halo_kernels_gemm_workspace_bytes).
OPERANDS_PACKED = 0
OPERANDS_FP6 = 1
# STREAM entries (block_m 16, 32, 64; block_k 32; csrc/shk_skinny.h) read the
# packed operands directly; per-channel calls split a tile's K over several
# workgroups when given a zero-filled workspace (every launch leaves what it
# used zero, counters and partials): sk_split_count / sk_workspace_bytes.
OPERANDS_STREAM = 2
FP6_MAX_K = 262144
# Largest K of the fp6 entries (32-bit buffer offsets of a tile's panels);
# per-channel calls with K > FP6_MAX_K run in exact K slices of FP6_MAX_K
# whose int32 sums add into the workspace, except on the persistent tile.
FP6_MAX_K_SLICED = 1 << 24
# Largest K per int32 accumulator of the int8 engines' int4 per-channel
# entries: products are widened x16, so |sum| <= 128 * 128 * K < 2^31 needs
# K < 131072 (K = 131072 overflows when every product is (-8) * (-8)).
INT4_ACC_MAX_K = 131071
# Bytes of the library's static scratch array (SHK_NOALLOC_SCRATCH_BYTES): the
# largest fp6 workspace amd_strix_halo_kernels_launch_gemm_noalloc accepts.
NOALLOC_SCRATCH_BYTES = 128 * 1024 * 1024

# Tile schedules (reference metadata.KernelSchedule): STANDARD launches one
# workgroup per tile, PERSISTENT one per resident slot, striding over tiles.
SCHEDULE_STANDARD = 0
SCHEDULE_PERSISTENT = 1

# Device quantization (amd_strix_halo_kernels_quantize): sources and outputs.
SRC_F32 = 0
SRC_F16 = 1
SRC_BF16 = 2
SRC_I8 = 3
QUANT_CODES = 0
QUANT_PACK_COLS = 1
QUANT_PACK_ROWS = 2


@dataclass(frozen=True)
class KernelDesc:
    """One entry of the library's kernel table (struct shk_kernel_desc)."""

    index: int
    family: int
    dtype_bits: int
    layout: int
    scale_mode: int
    min_subchannel: int
    max_subchannel: int
    epilogue_kind: int
    block_m: int
    block_n: int
    block_k: int
    num_waves: int
    num_stages: int
    lds_bytes: int
    group_size_m: int
    operand_format: int = OPERANDS_PACKED
    schedule: int = SCHEDULE_STANDARD
    split_k: int = 1

    @property
    def needs_workspace(self) -> bool:
        return self.operand_format == OPERANDS_FP6

    @property
    def is_stream(self) -> bool:
        return self.operand_format == OPERANDS_STREAM

    def workspace_bytes(self, m: int, n: int, k: int) -> int:
        """Bytes of the workspace for shape (m, n, k): fp6 operands (FP6;
        per-channel calls with K > FP6_MAX_K add [m, b_cols] int32 sums), the
        split-K counters and partials (STREAM), 0 for PACKED."""
        return _workspace_bytes(self, m, n, k)

    def _workspace_bytes(self, m: int, n: int, k: int) -> int:
        if self.is_stream:
            return sk_workspace_bytes(self, m, n, k)
        if not self.needs_workspace:
            return 0
        b_cols = 2 * n if self.epilogue_kind == EPI_KIND_SWIGLU else n
        nbytes = (m * k * 3) // 4 + (b_cols * k * 3) // 4
        if self.scale_mode == SCALE_PER_CHANNEL and k > FP6_MAX_K:
            nbytes += 4 * m * b_cols
        return nbytes

    @property
    def max_k(self) -> int | None:
        """Largest logical K a dense entry runs (None: no bound), as the
        library checks it (capi.hip dense_max_k)."""
        if self.family != FAMILY_DENSE:
            return None
        if self.is_stream:
            return FP6_MAX_K_SLICED if (self.dtype_bits == 4 and self.scale_mode == SCALE_PER_CHANNEL) else None
        if self.operand_format == OPERANDS_FP6:
            if self.scale_mode == SCALE_PER_CHANNEL and self.schedule == SCHEDULE_PERSISTENT:
                return FP6_MAX_K
            return FP6_MAX_K_SLICED
        if self.dtype_bits == 4 and self.scale_mode == SCALE_PER_CHANNEL:
            return INT4_ACC_MAX_K * max(1, self.split_k)
        return None

    def supports_k(self, k: int) -> bool:
        bound = self.max_k
        return bound is None or k <= bound

    def ragged_workspace_bytes(self, m: int, n: int, k_packed: int, groups: int) -> int:
        """Bytes of the operand workspace of a ragged call (0 for PACKED):
        with K rounded up to 128 (256 for the subchannel entries), the
        forward holds A (round32(m) rows) and per group B (round32(n) rows);
        the backward per group A, then per group B (k_f6ragged.hip)."""
        if not self.needs_workspace or m == 0 or n == 0 or groups == 0:
            return 0
        step = 256 if self.scale_mode == SCALE_SUBCHANNEL else 128
        kw = -(-2 * k_packed // step) * step
        m32, n32 = -(-m // 32) * 32, -(-n // 32) * 32
        if self.family == FAMILY_RAGGED_FWD:
            return (m32 * kw * 3) // 4 + groups * ((n32 * kw * 3) // 4)
        return groups * ((m32 * kw * 3) // 4 + (n32 * kw * 3) // 4)

    def serves_subchannel(self, size: int | None) -> bool:
        if self.scale_mode == SCALE_PER_CHANNEL:
            return size is None
        return size is not None and self.min_subchannel <= size <= self.max_subchannel


# The 32x32 engines (fp6 per-channel, int8 direct-to-LDS) keep each wave's
# 256 bytes of B scales in LDS past the stage ring (shk_f6.h).
MFMA32_SCALE_BYTES = 4 * 256

# Skinny (STREAM) tiles: 4 waves, wave-private rings of stages of 64 source
# bytes per row (shk_skinny.h); 64 output columns per-channel, 16 subchannel
# (the waves share the columns and take the scale groups in turn).
SK_NW = 4
SK_BN = 64
SK_BN_SUBCH = 16
SK_TARGET_UNITS = 256


def _sk_geometry(r: int, swiglu: bool, subch: bool) -> tuple[int, int]:
    """(ring depth, LDS bytes) of a skinny tile of r rows (SkCfg)."""
    bn = SK_BN_SUBCH if subch else SK_BN
    wcols = 2 * bn if swiglu else bn
    stage = r * 64 + wcols * 64 + ((r // 16) * 256 + 256 if subch else 0)
    tiles = (r // 16) * (wcols // 16)
    ch = (4 if tiles == 1 else 2 if tiles == 2 else 1) if subch else 0  # groups per wave and round
    chain = 2 * SK_NW * ch * tiles * 1024  # two rounds of scaled partials
    budget = 79872 - chain
    depth = 4 if SK_NW * 4 * stage <= budget else (3 if SK_NW * 3 * stage <= budget else 2)
    ring = SK_NW * depth * stage
    red = 0 if subch else SK_NW * (wcols // 16) * 1024
    return depth, max(ring, red) + chain


def sk_split_count(desc: "KernelDesc", m: int, n: int, k: int, with_workspace: bool = True) -> int:
    """Workgroups sharing a skinny per-channel tile's K (shk_table.h
    sk_split_count): about SK_TARGET_UNITS workgroups with at least two
    stages per wave, at most 16; for int4 enough to keep every wave within
    1023 stages of 128 K.  Without a workspace 1, or 0 if K needs a split."""
    if desc.scale_mode == SCALE_SUBCHANNEL:
        return 1
    ks = 128 if desc.dtype_bits == 4 else 64
    nst = -(-k // ks)
    need = 1
    if desc.dtype_bits == 4:
        while need * 4 * 1023 < nst:
            need *= 2
    if not with_workspace:
        return 1 if need == 1 else 0
    tiles = (m // desc.block_m) * (n // desc.block_n)
    s = 1
    while s * 2 <= 16 and tiles * s * 2 <= SK_TARGET_UNITS and nst >= 16 * s:
        s *= 2
    return max(s, need)


def sk_workspace_bytes(desc: "KernelDesc", m: int, n: int, k: int) -> int:
    """Arrival counters (padded to 256 bytes) and exact int32 partials of a
    split skinny launch; 0 when it runs unsplit (shk_table.h)."""
    s = sk_split_count(desc, m, n, k, True)
    if s <= 1:
        return 0
    tiles = (m // desc.block_m) * (n // desc.block_n)
    cf = 2 if desc.epilogue_kind == EPI_KIND_SWIGLU else 1
    return ((tiles * 4 + 255) & ~255) + tiles * s * (desc.block_n // 16) * (desc.block_m // 16) * cf * 1024


def _desc(index, family, bits, layout, *, bm, bn, bk, wm, wn, swiglu=False, subch=False, mk=64, group_m=8, pipe=0,
          fp6=False, fp6_sub=False, fp6_small=False, schedule=SCHEDULE_STANDARD, split_k=1):
    # pipe > 0: direct-to-LDS engine with a ring of `pipe` packed stages of 64
    # source bytes per tile row; 0: register-staged engine, two widened stages.
    # fp6: three stages of 256 A rows + 256 B rows x 128 K in fp6 (96 bytes).
    # fp6_sub: a 72 KiB ring of 128 + 128 rows in fp6 (96 bytes per 128 K) and
    # an eight-slot scale ring (shk_f6sub.h).  Groups of 256 run three 128-K
    # stage slots (the entry's num_stages, 3) and four 768-byte scale slots;
    # groups of 64 and 128 run six 64-K slots of the same ring, one or two per
    # group, and eight 768-byte scale slots; groups of 32 two per 64-K slot and
    # eight 1024-byte scale slots (two b_scale rows each), the entry's LDS.
    # fp6_small: two stages of 128 A rows + 128 B rows x 128 K in fp6 (96
    # bytes), then the B-scale slots (shk_f6small.h; k_f6ragged.hip).
    brows = 2 * bn if swiglu else bn
    if fp6_small:
        fp6 = True
        pipe = 2
        lds = pipe * (bm + bn) * 96 + MFMA32_SCALE_BYTES
    elif fp6_sub:
        fp6 = True
        pipe = 3
        lds = pipe * (bm + bn) * 96 + 8 * 1024
    elif fp6:
        pipe = 3
        lds = pipe * (bm + 256) * 96 + MFMA32_SCALE_BYTES
    else:
        lds = pipe * (bm + brows) * 64 if pipe else 2 * (bm * bk + brows * bk)
        if bits == 8 and pipe:
            lds += MFMA32_SCALE_BYTES
    return KernelDesc(
        index=index,
        family=family,
        dtype_bits=bits,
        layout=layout,
        scale_mode=SCALE_SUBCHANNEL if subch else SCALE_PER_CHANNEL,
        min_subchannel=(32 if mk == 32 or fp6_sub else 64) if subch else 0,
        max_subchannel=(32 if mk == 32 else 256) if subch else 0,
        epilogue_kind=EPI_KIND_SWIGLU if swiglu else EPI_KIND_PLAIN,
        block_m=bm,
        block_n=bn,
        block_k=bk,
        num_waves=wm * wn,
        num_stages=pipe or 2,
        lds_bytes=lds,
        group_size_m=group_m,
        operand_format=OPERANDS_FP6 if fp6 else OPERANDS_PACKED,
        schedule=schedule,
        split_k=split_k,
    )


def _sk_desc(index, bits, layout, r, *, swiglu=False, subch=False, schedule=SCHEDULE_STANDARD, split_k=1):
    depth, lds = _sk_geometry(r, swiglu, subch)
    return KernelDesc(
        index=index, family=FAMILY_DENSE, dtype_bits=bits, layout=layout,
        scale_mode=SCALE_SUBCHANNEL if subch else SCALE_PER_CHANNEL,
        min_subchannel=32 if subch else 0, max_subchannel=256 if subch else 0,
        epilogue_kind=EPI_KIND_SWIGLU if swiglu else EPI_KIND_PLAIN,
        block_m=r, block_n=SK_BN_SUBCH if subch else SK_BN, block_k=32, num_waves=SK_NW, num_stages=depth,
        lds_bytes=lds,
        group_size_m=1, operand_format=OPERANDS_STREAM, schedule=schedule, split_k=split_k)


def _build() -> tuple[KernelDesc, ...]:
    out: list[KernelDesc] = []

    def add(**kw):
        out.append(_desc(len(out), **kw))

    def add_sk(*args, **kw):
        out.append(_sk_desc(len(out), *args, **kw))

    for bits in (4, 8):
        big_bk = 128 if bits == 4 else 64
        for layout in (LAYOUT_NN, LAYOUT_NT, LAYOUT_TN):
            d = dict(family=FAMILY_DENSE, bits=bits, layout=layout)
            if bits == 4:
                add(**d, bm=256, bn=256, bk=128, wm=2, wn=2, fp6=True)
                add(**d, bm=256, bn=128, bk=128, wm=2, wn=2, swiglu=True, fp6=True)
                add(**d, bm=128, bn=128, bk=128, wm=2, wn=2, subch=True, fp6_sub=True)
            add(**d, bm=256, bn=256, bk=big_bk, wm=2, wn=2, pipe=4)
            add(**d, bm=256, bn=128, bk=big_bk, wm=2, wn=2, swiglu=True, pipe=4)
            add(**d, bm=128, bn=128, bk=64, wm=2, wn=2)
            add(**d, bm=64, bn=64, bk=64, wm=2, wn=2)
            add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, swiglu=True)
            add(**d, bm=256, bn=128, bk=big_bk, wm=4, wn=2, subch=True)
            add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, subch=True)
            add(**d, bm=256, bn=64, bk=big_bk, wm=4, wn=2, swiglu=True, subch=True)
            add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, swiglu=True, subch=True)
            add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, subch=True, mk=32)
            add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, swiglu=True, subch=True, mk=32)
    for layout in (LAYOUT_NN, LAYOUT_NT, LAYOUT_TN, LAYOUT_TT):
        # fp6 entries lead each family (k_ragged.hip)
        add(family=FAMILY_RAGGED_FWD, bits=4, layout=layout, group_m=1, bm=128, bn=128, bk=128, wm=2, wn=2,
            fp6_small=True)
        add(family=FAMILY_RAGGED_FWD, bits=4, layout=layout, group_m=1, bm=128, bn=128, bk=128, wm=2, wn=2,
            subch=True, fp6_sub=True)
        for subch, mk in ((False, 64), (True, 64), (True, 32)):
            f = dict(family=FAMILY_RAGGED_FWD, bits=4, layout=layout, subch=subch, mk=mk, group_m=1)
            add(**f, bm=16, bn=128, bk=128, wm=1, wn=4)
            add(**f, bm=32, bn=128, bk=128, wm=2, wn=2)
            add(**f, bm=64, bn=128, bk=128, wm=2, wn=2)
            add(**f, bm=128, bn=128, bk=128, wm=2, wn=2)
        add(family=FAMILY_RAGGED_BWD, bits=4, layout=layout, group_m=1, bm=128, bn=128, bk=128, wm=2, wn=2,
            fp6_small=True)
        add(family=FAMILY_RAGGED_BWD, bits=4, layout=layout, group_m=1, bm=128, bn=128, bk=128, wm=2, wn=2,
            subch=True, fp6_sub=True)
        for subch, mk in ((False, 64), (True, 64), (True, 32)):
            add(family=FAMILY_RAGGED_BWD, bits=4, layout=layout, subch=subch, mk=mk, group_m=1, bm=128, bn=128,
                bk=128, wm=2, wn=2)
    # persistent int4 entries (plain epilogue kind) after the ragged families
    for layout in (LAYOUT_NN, LAYOUT_NT, LAYOUT_TN):
        d = dict(family=FAMILY_DENSE, bits=4, layout=layout, schedule=SCHEDULE_PERSISTENT)
        add(**d, bm=256, bn=256, bk=128, wm=2, wn=2, fp6=True)
        add(**d, bm=128, bn=128, bk=128, wm=2, wn=2, subch=True, fp6_sub=True)
        add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, subch=True)
        add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, subch=True, mk=32)
    # split-K 2/4/8 (fp32 output): 128x128 per-channel, int4 64x64 subchannel
    for bits in (4, 8):
        for layout in (LAYOUT_NN, LAYOUT_NT, LAYOUT_TN):
            d = dict(family=FAMILY_DENSE, bits=bits, layout=layout)
            for split in (2, 4, 8):
                add(**d, bm=128, bn=128, bk=64, wm=2, wn=2, split_k=split)
            if bits == 4:
                for mk in (64, 32):
                    for split in (2, 4, 8):
                        add(**d, bm=64, bn=64, bk=64, wm=2, wn=2, subch=True, mk=mk, split_k=split)
    # skinny tiles (k_skinny.hip), per (bits, layout)
    for bits in (4, 8):
        for layout in (LAYOUT_NN, LAYOUT_NT, LAYOUT_TN):
            for r in (16, 32, 64):
                for swiglu, subch in ((False, False), (True, False), (False, True), (True, True)):
                    add_sk(bits, layout, r, swiglu=swiglu, subch=subch)
            if bits == 4:
                for split in (1, 2, 4, 8):
                    for r in (16, 32, 64):
                        for subch in (False, True):
                            add_sk(bits, layout, r, subch=subch, schedule=SCHEDULE_PERSISTENT, split_k=split)
            for split in (2, 4, 8):
                for r in (16, 32, 64):
                    for subch in (False, True):
                        add_sk(bits, layout, r, subch=subch, split_k=split)
    return tuple(out)


TABLE: tuple[KernelDesc, ...] = _build()


@functools.lru_cache(maxsize=4096)
def _workspace_bytes(desc: KernelDesc, m: int, n: int, k: int) -> int:
    # memoized: mm() sizes the workspace on every call
    return desc._workspace_bytes(m, n, k)


def measured_tops(desc: KernelDesc) -> float | None:
    """Throughput measured on MI355X (bench.py and sweeps on one GPU; the
    whole call including operand conversion), used by the registry's
    selection like the reference's benchmark TOPS (registry.py:254-352):
    fp6 int4 per-channel 256x256 (C2, 8192^3), fp6 int4 SwiGLU 256x128
    (4096 x 2*11008 x 4096), fp6 int4 subchannel 128x128 (C3), int8 32x32
    SwiGLU 256x128 (C4) and int8 plain 256x256 (8192^3), and the skinny
    tiles (SKINNY_TOPS, SKINNY_SUB_TOPS).  Other entries have no measurement
    and rank by tile area."""
    if desc.family != FAMILY_DENSE or desc.schedule != SCHEDULE_STANDARD or desc.split_k > 1:
        return None
    if desc.operand_format == OPERANDS_FP6:
        if desc.scale_mode == SCALE_SUBCHANNEL:
            return 2001.0
        return 3504.0 if desc.epilogue_kind == EPI_KIND_PLAIN else 3161.0
    if desc.operand_format == OPERANDS_STREAM:
        return SKINNY_TOPS if desc.scale_mode == SCALE_PER_CHANNEL else SKINNY_SUB_TOPS[desc.block_m]
    if desc.dtype_bits == 8 and desc.num_stages == 4 and desc.block_m == 256:
        return 2014.0 if desc.epilogue_kind == EPI_KIND_SWIGLU else 2270.0
    return None


# The skinny per-channel tiles' figure: the bench's skinny line (int4, M = 16,
# N = K = 8192, 8.9 us per launch: 241 TOPS).  int8 and SwiGLU skinny tiles
# carry it too: at N = K = 4096 and M = 64 to 4160 every skinny per-channel
# tile (int4 and int8, plain and SwiGLU) ran 1.2-3x faster than the
# register-staged 64x64 and 128x128 tiles, which outranked it by area.  The
# larger measured tiles keep their higher figures where they fit.
SKINNY_TOPS = 241.0

# The skinny subchannel tiles' figures by tile height: int4, N = K = 8192,
# groups of 128; 16 rows at M = 16 (22.3 us, 96 TOPS), 32 and 64 rows at
# M = 64 (46.6 and 56.6 us: 184 and 152 TOPS), so the 32-row tile, the
# fastest of them at M = 64 and 192, ranks first where it fits.  They rank
# above the register-staged subchannel tiles up to M = SKINNY_SUB_MAX_M rows:
# at N = K = 4096 they ran 3x faster at M = 64 and 1.0-1.4x at M = 192, and
# from M = 576 up to 1.8x slower (groups of 32 from M = 320).
SKINNY_SUB_TOPS = {16: 96.0, 32: 184.0, 64: 152.0}
SKINNY_SUB_MAX_M = 256


def selection_tops(desc: KernelDesc, m: int) -> float | None:
    """measured_tops as select ranks an entry for M rows (capi.hip
    measured_score): the skinny subchannel tiles' figure holds up to
    SKINNY_SUB_MAX_M rows."""
    tops = measured_tops(desc)
    if (tops is not None and desc.operand_format == OPERANDS_STREAM and desc.scale_mode == SCALE_SUBCHANNEL
            and m > SKINNY_SUB_MAX_M):
        return None
    return tops


def entries(family: int) -> tuple[KernelDesc, ...]:
    return tuple(d for d in TABLE if d.family == family)


@functools.lru_cache(maxsize=None)
def ragged_task_capacity(rows: int, groups: int, tile: int) -> int:
    """Upper bound on the row tasks of `rows` rows in `groups` groups with
    tasks of `tile` rows (amd_strix_halo_kernels_ragged_task_capacity): every
    group adds at most one partial task at each end."""
    if rows < 0 or groups < 0 or tile <= 0:
        return 0
    return min(rows // tile + 2 * groups + 1, 0x7FFFFFFF)


@functools.lru_cache(maxsize=None)
def find_ragged(family: int, *, layout: int, subchannel: int | None, block_m: int | None = None,
                fp6: bool = False) -> KernelDesc:
    """Ragged kernel for a layout and scale mode (and task rows for the
    forward): an FP6 entry if `fp6`, else one that reads the packed operands."""
    fmt = OPERANDS_FP6 if fp6 else OPERANDS_PACKED
    for d in TABLE:
        if d.family != family or d.layout != layout or not d.serves_subchannel(subchannel):
            continue
        if d.operand_format != fmt:
            continue
        if block_m is not None and d.block_m != block_m:
            continue
        return d
    raise LookupError(
        f"no gfx950 ragged kernel for family={family}, layout={layout}, subchannel={subchannel}, block_m={block_m}, "
        f"fp6={fp6}"
    )


def ragged_fp6_eligible(family: int, *, subchannel: int | None, m: int, n: int, k_packed: int) -> bool:
    """Whether a ragged call's sizes suit the fp6 entries (k_f6ragged.hip):
    N a multiple of 8 (whole 16-byte output units) and K at most FP6_MAX_K;
    per-channel, or subchannel with M * ceil(K/S) even (the tile reads
    a_scale in whole dwords; groups of 32 in pairs, so ceil(K/32) even)."""
    if subchannel is not None:
        cols = -(-2 * k_packed // subchannel)
        if m * cols % 2 or (subchannel == 32 and cols % 2):
            return False
    return n % 8 == 0 and 2 * k_packed <= FP6_MAX_K


# Task rows of the forward kernels that read packed operands, and of the fp6
# forward (whose task list is built with align_tile 32).
RAGGED_FWD_BLOCK_M = tuple(sorted({d.block_m for d in entries(FAMILY_RAGGED_FWD) if not d.needs_workspace}))
RAGGED_FP6_BLOCK_M = 128
# RaggedDotConfig.block_m that asks for the fp6 forward (as does the default,
# 64, where the fp6 kernel applies); the other heights pick the packed kernels.
RAGGED_FP6_CONFIG_BLOCK_M = 256
RAGGED_FP6_ALIGN = 32
