"""``asc.lib.host``: the host matmul tiling API (python/asc/lib/host/wrappers.py).

On the reference these classes are bindings to the CANN tiling library, which
splits a matmul over Ascend cube cores and fills a ``TCubeTiling`` for the kernel
(python/tutorials/03_matmul_mix/matmul_mix.py:90-106,
04_matmul_cube_only/matmul_cube_only.py:97-115).  The split algorithm lives in
CANN, not in the reference, and the MI355X kernels choose their own tiles, so the
split here is build-defined: it only has to describe a launch that covers the whole
output.  ``set_dim(n)`` gives the number of kernel instances the split may use
(``used_core_num`` <= n); a mixed cube + vector kernel runs two instances per launched
block, which is why the tutorials launch ``used_core_num // 2`` or ``dim // 2`` blocks
(matmul_leakyrelu.py:92, matmul_mix.py:86).  N is split first, then M, in multiples
of 16, or as ``set_single_shape`` / ``set_fix_split`` ask.  The other setters record
their values and return 0, as the reference's return codes do on success.
"""
from __future__ import annotations

from enum import Enum
from typing import Optional


class TPosition(Enum):
    GM = 0
    A1 = 1
    A2 = 2
    B1 = 3
    B2 = 4
    C1 = 5
    C2 = 6
    CO1 = 7
    CO2 = 8
    VECIN = 9
    VECOUT = 10
    VECCALC = 11
    LCM = 12
    SPM = 13
    SHM = 14
    TSCM = 15
    MAX = 16


class CubeFormat(Enum):
    ND = 0
    NZ = 1
    ZN = 2
    ZZ = 3
    NN = 4
    ND_ALIGN = 5
    SCALAR = 6
    VECTOR = 7
    ROW_MAJOR = 8
    COLUMN_MAJOR = 9


class DataType(Enum):
    DT_FLOAT = 0
    DT_FLOAT16 = 1
    DT_INT8 = 2
    DT_INT32 = 3
    DT_UINT8 = 4
    DT_INT16 = 6
    DT_UINT16 = 7
    DT_UINT32 = 8
    DT_INT64 = 9
    DT_UINT64 = 10
    DT_DOUBLE = 11
    DT_BOOL = 12
    DT_BF16 = 27
    DT_BFLOAT16 = 27  # alias of DT_BF16


class MatrixTraverse(Enum):
    NOSET = 0
    FIRSTM = 1
    FIRSTN = 2


class MatrixMadType(Enum):
    NORMAL = 0
    HF32 = 1


class Platform:
    """The device the tiling is made for (the reference's PlatformAscendC)."""

    def __init__(self, core_num: int):
        self.core_num = core_num

    def get_core_num(self) -> int:
        return self.core_num


def get_ascendc_platform() -> Platform:
    """The current device's platform: its compute-unit count (256 on MI355X)."""
    try:
        from ... import _native
        return Platform(int(_native.device_info(0)["cu_count"]))
    except Exception:  # no device visible: the tiling needs only the MI355X count
        return Platform(256)


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


class MatmulApiTiling:
    """Single-core tiling (the reference's MatmulApiTiling): one block computes everything."""

    def __init__(self, platform: Optional[Platform] = None):
        self.platform = platform or get_ascendc_platform()
        self.types = {}
        self.m = self.n = self.k = None
        self.org = None
        self.is_bias = False
        self.dim = 1

    def _set_type(self, which: str, pos, fmt, dtype, is_trans: bool = False) -> int:
        self.types[which] = (pos, fmt, dtype, bool(is_trans))
        return 0

    def set_a_type(self, pos, type, data_type, is_trans: bool = False) -> int:  # noqa: A002
        return self._set_type("a", pos, type, data_type, is_trans)

    def set_b_type(self, pos, type, data_type, is_trans: bool = False) -> int:  # noqa: A002
        return self._set_type("b", pos, type, data_type, is_trans)

    def set_c_type(self, pos, type, data_type) -> int:  # noqa: A002
        return self._set_type("c", pos, type, data_type)

    def set_bias_type(self, pos, type, data_type) -> int:  # noqa: A002
        return self._set_type("bias", pos, type, data_type)

    def set_org_shape(self, org_m: int, org_n: int, org_ka: int, org_kb: Optional[int] = None) -> int:
        self.org = (int(org_m), int(org_n), int(org_ka), int(org_ka if org_kb is None else org_kb))
        return 0

    def set_shape(self, m: int, n: int, k: int) -> int:
        self.m, self.n, self.k = int(m), int(n), int(k)
        return 0

    def enable_bias(self, is_bias_in: bool = False) -> int:
        self.is_bias = bool(is_bias_in)
        return 0

    def set_buffer_space(self, l1_size: int = -1, l0_c_size: int = -1, ub_size: int = -1, bt_size: int = -1) -> int:
        return 0

    def set_traverse(self, traverse) -> int:
        self.traverse = traverse
        return 0

    def set_fix_split(self, base_m_in: int = -1, base_n_in: int = -1, base_k_in: int = -1) -> int:
        self.fix_split = (int(base_m_in), int(base_n_in), int(base_k_in))
        return 0

    def set_double_buffer(self, a: bool, b: bool, c: bool, bias: bool, trans_nd2nz: bool = True,
                          trans_nz2nd: bool = True) -> int:
        return 0

    def set_mad_type(self, mad_type) -> int:
        return 0

    def set_split_range(self, *args, **kwargs) -> int:
        return 0

    def set_a_layout(self, b: int, s: int, n: int, g: int, d: int) -> int:
        self.a_layout = (int(b), int(s), int(n), int(g), int(d))
        return 0

    def set_b_layout(self, b: int, s: int, n: int, g: int, d: int) -> int:
        self.b_layout = (int(b), int(s), int(n), int(g), int(d))
        return 0

    def set_c_layout(self, b: int, s: int, n: int, g: int, d: int) -> int:
        self.c_layout = (int(b), int(s), int(n), int(g), int(d))
        return 0

    def set_batch_num(self, batch: int) -> int:
        self.batch_num = int(batch)
        return 0

    def set_batch_info_for_normal(self, batch_a: int, batch_b: int, m: int, n: int, k: int) -> int:
        self.set_a_layout(batch_a, m, 1, 1, k)
        self.set_b_layout(batch_b, k, 1, 1, n)
        self.set_c_layout(max(int(batch_a), int(batch_b)), m, 1, 1, n)
        return 0

    def set_matmul_config_params(self, *args, **kwargs) -> int:
        return 0

    def _split(self):
        return self.m, self.n, 1

    def get_tiling(self, tiling) -> int:
        """Fills ``tiling`` (an asc.adv.TCubeTiling); returns 0, or -1 without a shape."""
        if self.m is None:
            if self.org is None:
                return -1
            self.m, self.n, self.k = self.org[0], self.org[1], self.org[2]
        for v, name in ((self.m, "m"), (self.n, "n"), (self.k, "k")):
            if v <= 0:
                raise ValueError(f"matmul tiling: {name} must be positive, got {v}")
        org = self.org or (self.m, self.n, self.k, self.k)
        single_m, single_n, used = self._split()
        fix_m, fix_n, fix_k = getattr(self, "fix_split", (-1, -1, -1))
        base_m = fix_m if fix_m > 0 else min(single_m, 256)
        base_n = fix_n if fix_n > 0 else min(single_n, 256)
        base_k = fix_k if fix_k > 0 else min(self.k, 64)
        fields = dict(used_core_num=used, m=self.m, n=self.n, k_a=self.k, k_b=self.k, org_m=org[0], org_n=org[1],
                      org_ka=org[2], org_kb=org[3], single_core_m=single_m, single_core_n=single_n,
                      single_core_k=self.k, base_m=base_m, base_n=base_n, base_k=base_k, depth_a1=1, depth_b1=1,
                      step_m=1, step_n=1, step_ka=1, step_kb=1, is_bias=int(self.is_bias), share_mode=0)
        # batch layouts (TCubeTiling's ALayoutInfo* / BLayoutInfo* / CLayoutInfo* / BatchNum;
        # -1 when not set, as the struct's defaults, python/asc/language/adv/tiling.py:45-60)
        for prefix, names, layout in (("a", "bsngd", getattr(self, "a_layout", None)),
                                      ("b", "bsngd", getattr(self, "b_layout", None)),
                                      ("c", ("b", "s1", "n", "g", "s2"), getattr(self, "c_layout", None))):
            for i, name in enumerate(names):
                fields[f"{prefix}_layout_info_{name}"] = layout[i] if layout else -1
        fields["batch_num"] = getattr(self, "batch_num", -1)
        for key, value in fields.items():
            setattr(tiling, key, value)
        return 0


class MultiCoreMatmulTiling(MatmulApiTiling):
    """Multi-core tiling: the output split over at most ``dim`` instances."""

    def __init__(self, platform: Optional[Platform] = None):
        super().__init__(platform)
        self.dim = self.platform.get_core_num()
        self.single_shape = None

    def set_dim(self, dim: int) -> int:
        if int(dim) <= 0:
            raise ValueError(f"set_dim: the core count must be positive, got {dim}")
        self.dim = int(dim)
        return 0

    def set_single_shape(self, single_m_in: int = -1, single_n_in: int = -1, single_k_in: int = -1) -> int:
        self.single_shape = (int(single_m_in), int(single_n_in))
        return 0

    def enable_multi_core_split_k(self, flag: bool) -> None:
        if flag:
            raise NotImplementedError("a split over K is not provided: each instance takes the full K")

    def _split(self):
        if self.single_shape is not None and min(self.single_shape) > 0:
            sm, sn = self.single_shape
            return sm, sn, -(-self.m // sm) * -(-self.n // sn)
        blocks = self.dim
        single_n = min(_round_up(-(-self.n // blocks), 16), _round_up(self.n, 16))
        n_blocks = -(-self.n // single_n)
        m_blocks = max(1, min(blocks // n_blocks, -(-self.m // 16)))
        single_m = _round_up(-(-self.m // m_blocks), 16)
        m_blocks = -(-self.m // single_m)
        return single_m, single_n, m_blocks * n_blocks

    def get_core_num(self) -> int:
        return self.dim
