"""Host-side launch planner for ``pth_flash_attn_fwd`` on MI355X (gfx950).

Drop-in for the reference planner (``python/pth_flash_attn/planner.py``): the
same functions, keyword-only parameters, ``LaunchPlan`` fields, error types and
formulas (reference planner.py:24-73). Only the kernel-trait constants are
re-derived for the gfx950 kernels of this package.

Why it takes host ints only: a HIP graph captures one grid per padded batch
descriptor and replays it while the sequence lengths grow on the device, so no
output here may depend on a length. No parameter can carry one: every
parameter is keyword-only, must be a real ``int``/``bool`` (a 0-d tensor is
refused: it would force a device-to-host sync), and the device's CU count is
an input, never a query. The module imports only the standard library.

Formulas (G = Hq / Hkv, b_max = 64 // G query tokens per 64-row tile):

decode-like launch::

    rt = ceil(q_max / b_max)                 row tiles per request
    wm = smallest of {1, 2, 4} with 16 wm >= ceil(q_max / rt) * G
    bq = floor(16 wm / G)
    S  = ceil(C_target / (Hkv * rt))         one request alone fills the GPU

prefill launch::

    wm = 4, bq = b_max, S = ceil(C_target / (Hkv * ceil(T / bq)))

both::

    C_target      = num_sms * CTAS_PER_SM[D]
    S             = clamp(S, 1, ws_token_splits // T)
    window W > 0: S = min(S, ceil((W + q_max - 2) / 64) + 1)
    q_tiles_upper = T // bq + num_reqs

MI355X constants. A "CTA" of the formulas is one work unit of the gfx950
kernel: (row tile, KV head, 16-row group, split), run by one wave64. The D=128
kernel holds 2 waves per SIMD (<= 256 VGPRs), 4 SIMDs per CU, so one CU keeps
8 units resident: CTAS_PER_SM[128] = 8 and C_target = 256 CUs * 8 = 2048 on
MI355X. The kernel itself uses only as many of the S splits as a row tile's
length needs (read on the device; at least one 32-key chunk per split), so a large S
costs empty work-groups, not combine traffic. D = 64 and 256 run on the
register-load kernel (8 waves per CU as well). Their entries only size the
split count: 8 for D = 64; 4 for D = 256, whose units read twice the bytes per
key, so half as many splits already keep the CUs' loads in flight.
"""

from __future__ import annotations

from dataclasses import dataclass

# Query rows per 16x16 MFMA column block: one wave owns 16 query rows.
MMA_ROWS_PER_WARP = 16
# Row-tile heights the op accepts, in units of 16 rows.
WM_CHOICES = (1, 2, 4)
# Rows per row tile = 64; also the GQA packing limit G <= 64.
MAX_ROWS_PER_CTA = MMA_ROWS_PER_WARP * WM_CHOICES[-1]
# Work units (waves) one CU keeps resident, by head size (see module docstring).
CTAS_PER_SM = {64: 8, 128: 8, 256: 4}
SUPPORTED_HEAD_SIZES = tuple(sorted(CTAS_PER_SM))
# Head size with a windowed / non-causal kernel.
WINDOWED_HEAD_SIZES = (128,)
# KV tokens per tile: the unit of the split partition.
KV_TILE_TOKENS = 64
# Split partials (O and log2-LSE) are fp32.
PARTIAL_BYTES_PER_ELEMENT = 4

# The only parameters plan_launch accepts, in order.
DESCRIPTOR_FIELDS = (
    "num_tokens",
    "num_reqs",
    "max_query_len",
    "G",
    "Hkv",
    "D",
    "num_sms",
    "is_prefill",
    "ws_token_splits",
    "window",
)


def _cdiv(a: int, b: int) -> int:
    """Integer ceil(a / b) for a >= 0, b > 0 (exact at any size)."""
    return -(-a // b)


def _host_int(name: str, value: object, minimum: int) -> int:
    """Return value if it is a plain int (not bool) >= minimum, else raise."""
    if isinstance(value, bool) or not isinstance(value, int):
        raise TypeError(f"{name} must be a host int, got {type(value).__name__}")
    if value < minimum:
        raise ValueError(f"{name} must be >= {minimum}, got {value}")
    return value


def _head_size(D: object) -> int:
    d = _host_int("D", D, 1)
    if d not in CTAS_PER_SM:
        raise ValueError(f"D must be one of {SUPPORTED_HEAD_SIZES}, got {d}")
    return d


def _group(G: object) -> int:
    g = _host_int("G", G, 1)
    if g > MAX_ROWS_PER_CTA:
        raise ValueError(f"G must be <= {MAX_ROWS_PER_CTA}, got {g}")
    return g


def c_target(*, D: int, num_sms: int) -> int:
    """Work units that fill the GPU once: num_sms * CTAS_PER_SM[D]."""
    return _host_int("num_sms", num_sms, 1) * CTAS_PER_SM[_head_size(D)]


def max_tokens_per_tile(G: int) -> int:
    """b_max = 64 // G: query tokens of one request in a 64-row tile.

    Also the base of vLLM's decode (reorder) threshold.
    """
    return MAX_ROWS_PER_CTA // _group(G)


def wm_for_rows(rows: int) -> int:
    """Smallest wm in {1, 2, 4} with 16 * wm >= rows."""
    r = _host_int("rows", rows, 1)
    for wm in WM_CHOICES:
        if MMA_ROWS_PER_WARP * wm >= r:
            return wm
    raise ValueError(f"{r} rows exceed one {MAX_ROWS_PER_CTA}-row CTA tile")


def split_tile_range(*, split: int, num_splits: int, num_tiles: int) -> tuple[int, int]:
    """KV-tile range [start, end) of split ``split``: [s T / S, (s + 1) T / S).

    Ranges are disjoint, cover [0, T) and differ by at most one tile; when
    T < S some are empty. This is the reference's per-row-tile partition,
    kept as its interface; the gfx950 kernels cut the chunk streams of all
    row tiles into equal ranges per work-group instead (at most S per row
    tile).
    """
    total = _host_int("num_splits", num_splits, 1)
    s = _host_int("split", split, 0)
    tiles = _host_int("num_tiles", num_tiles, 0)
    if s >= total:
        raise ValueError(f"split {s} out of range for num_splits={total}")
    return (s * tiles) // total, ((s + 1) * tiles) // total


@dataclass(frozen=True)
class LaunchPlan:
    """The host side of one ``pth_flash_attn_fwd`` launch.

    wm, bq, q_tiles_upper and num_splits are the interface to the op; the rest
    records the descriptor the plan was made for.
    """

    wm: int
    bq: int
    q_tiles_upper: int
    num_splits: int
    num_tokens: int
    G: int
    Hkv: int
    D: int
    is_prefill: bool

    @property
    def Hq(self) -> int:
        """Query heads, G * Hkv."""
        return self.G * self.Hkv

    @property
    def rows_per_cta(self) -> int:
        """Query rows of one row tile: bq * G (<= 16 * wm)."""
        return self.bq * self.G

    @property
    def grid(self) -> tuple[int, int, int]:
        """(row-tile upper bound, KV heads, splits) of the planning model."""
        return (self.q_tiles_upper, self.Hkv, self.num_splits)

    @property
    def ws_token_splits_used(self) -> int:
        """Token-splits of workspace the launch writes (0 when S == 1)."""
        return self.num_splits * self.num_tokens if self.num_splits > 1 else 0

    @property
    def ws_o_shape(self) -> tuple[int, int, int, int]:
        """[S, T, Hq, D] fp32 partials to pass; S = 0 when S == 1."""
        s = self.num_splits if self.num_splits > 1 else 0
        return (s, self.num_tokens, self.Hq, self.D)

    @property
    def ws_lse_shape(self) -> tuple[int, int, int]:
        """[S, T, Hq] fp32 log2-LSE partials to pass; S = 0 when S == 1."""
        s = self.num_splits if self.num_splits > 1 else 0
        return (s, self.num_tokens, self.Hq)


def plan_launch(
    *,
    num_tokens: int,
    num_reqs: int,
    max_query_len: int,
    G: int,
    Hkv: int,
    D: int,
    num_sms: int,
    is_prefill: bool,
    ws_token_splits: int,
    window: int = 0,
) -> LaunchPlan:
    """Plan one launch from the padded batch descriptor of its slice.

    There is no sequence-length parameter: the plan is a pure function of
    these host integers, so a captured graph stays valid as lengths grow.
    ``num_sms`` is the device's compute-unit count (256 on MI355X).
    """
    t = _host_int("num_tokens", num_tokens, 1)
    reqs = _host_int("num_reqs", num_reqs, 1)
    q_max = _host_int("max_query_len", max_query_len, 1)
    g = _group(G)
    hkv = _host_int("Hkv", Hkv, 1)
    d = _head_size(D)
    sms = _host_int("num_sms", num_sms, 1)
    w_ts = _host_int("ws_token_splits", ws_token_splits, 0)
    w = _host_int("window", window, 0)
    if not isinstance(is_prefill, bool):
        raise TypeError(f"is_prefill must be a bool, got {type(is_prefill).__name__}")
    if q_max > t:
        raise ValueError(f"max_query_len={q_max} > num_tokens={t}")
    if t > reqs * q_max:
        raise ValueError(
            f"num_tokens={t} cannot come from {reqs} requests of at most {q_max} tokens"
        )

    b_max = max_tokens_per_tile(g)
    if is_prefill:
        wm = WM_CHOICES[-1]
        row_tiles = _cdiv(t, b_max)  # lower bound of sum_i ceil(q_i / bq)
    else:
        # Per request: a lone long request must fill the GPU by itself.
        row_tiles = _cdiv(q_max, b_max)
        wm = wm_for_rows(_cdiv(q_max, row_tiles) * g)
    bq = MMA_ROWS_PER_WARP * wm // g

    splits = _cdiv(c_target(D=d, num_sms=sms), hkv * row_tiles)
    splits = max(1, min(splits, w_ts // t))
    if w > 0:
        # A row tile sees at most W + q_max - 1 keys: at most
        # ceil((W + q_max - 2) / 64) + 1 KV tiles at the worst alignment.
        splits = min(splits, _cdiv(w + q_max - 2, KV_TILE_TOKENS) + 1)

    return LaunchPlan(
        wm=wm,
        bq=bq,
        q_tiles_upper=t // bq + reqs,
        num_splits=splits,
        num_tokens=t,
        G=g,
        Hkv=hkv,
        D=d,
        is_prefill=is_prefill,
    )


def s_alone(*, Hkv: int, D: int, num_sms: int) -> int:
    """Splits that let one row tile fill the GPU: ceil(C_target / Hkv)."""
    hkv = _host_int("Hkv", Hkv, 1)
    return _cdiv(c_target(D=D, num_sms=num_sms), hkv)


def workspace_token_splits(
    *, max_num_seqs: int, q_dec_max: int, Hkv: int, D: int, num_sms: int
) -> int:
    """W_ts = min(max_num_seqs, S_alone) * q_dec_max * S_alone token-splits."""
    seqs = _host_int("max_num_seqs", max_num_seqs, 1)
    q_dec = _host_int("q_dec_max", q_dec_max, 1)
    alone = s_alone(Hkv=Hkv, D=D, num_sms=num_sms)
    return min(seqs, alone) * q_dec * alone


def workspace_shapes(
    *, ws_token_splits: int, Hq: int, D: int
) -> tuple[tuple[int, int, int], tuple[int, int]]:
    """fp32 shapes to reserve once: O partials (W_ts, Hq, D), LSE (W_ts, Hq)."""
    w_ts = _host_int("ws_token_splits", ws_token_splits, 0)
    hq = _host_int("Hq", Hq, 1)
    d = _head_size(D)
    return (w_ts, hq, d), (w_ts, hq)


def workspace_bytes(*, ws_token_splits: int, Hq: int, D: int) -> int:
    """W_ts * Hq * (D + 1) * 4: bytes of both fp32 partial buffers."""
    (w_ts, hq, d), _ = workspace_shapes(ws_token_splits=ws_token_splits, Hq=Hq, D=D)
    return w_ts * hq * (d + 1) * PARTIAL_BYTES_PER_ELEMENT
