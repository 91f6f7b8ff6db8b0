"""CPU checks of the C ABI: the library builds and loads, exports exactly the entry points that
include/rus_amd.h declares, and rejects invalid arguments before touching the GPU."""

from __future__ import annotations

import ctypes

import re
import subprocess
from pathlib import Path

import pytest

from rus_amd import _lib

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "rus_amd.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(rus_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    assert lib.rus_abi_version() == _lib.ABI_VERSION
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (rus_[a-z0-9_]+)$", out, flags=re.M))
    declared = _declared()
    assert declared, "no declarations parsed from include/rus_amd.h"
    assert declared == exported
    # every declared compute entry point has a ctypes signature
    assert declared - {"rus_last_error", "rus_abi_version"} == set(_lib.SIGNATURES)


def test_header_compiles_as_c():
    src = '#include "rus_amd.h"\nint main(void){return RUS_OK;}\n'
    res = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{REPO / 'include'}", "-x", "c",
                          "-", "-o", "/dev/null"], input=src, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


@pytest.mark.parametrize(
    "name,args,msg",
    [
        # n_bytes beyond 2^31
        ("rus_nf4_dequant", (1, 1, 1, 1, 0.0, 0.0, 0.0, 0, 0, 0, 0, 1 << 31, 1, 1, 64, 256, 16, None),
         "n_bytes"),
        # blocksize not a power of two
        ("rus_nf4_dequant", (16, 16, 16, 16, 0.0, 0.0, 0.0, 64, 64, 0, 0, 64, 4, 1, 48, 256, 16, None),
         "blocksize"),
        # absmax too short for the bytes
        ("rus_nf4_dequant", (16, 16, 16, 16, 0.0, 0.0, 0.0, 64, 64, 0, 0, 64, 1, 1, 64, 256, 16, None),
         "absmax"),
        ("rus_nf4_dequant_multi", (None, 0, 16, 64, 256, None), "n_jobs"),
        # stride smaller than the row
        ("rus_rmsnorm_fwd", (16, None, 16, 0, None, 16, 16, 4, 128, 64, 1e-6, 0, None), "stride"),
        # bad dtype
        ("rus_rmsnorm_bwd", (16, 16, 16, 0, 16, None, 16, 4, 128, 128, 7, None), "dtype"),
        # head_dim not a multiple of 16
        ("rus_qkv_lora_rope_fwd", (16, None, None, 16, 16, 16, 16, 16, 16, 4, 2000, 0, 0, 120, 8,
                                   1.0, 1.0, 12, 2, 120, None, 0, None), "head_dim"),
        # only one of the LoRA gradients requested
        ("rus_qkv_rope_bwd", (16, 16, 16, 16, 16, 16, 16, 16, None, 4, 2048, 128, 8, 1.0, 1.0, 12,
                              2, 128, None, 0, None), "both"),
        ("rus_swiglu_fwd", (16, 16, 16, 4, 100, 50, 100, 100, 0, None), "stride"),
        ("rus_swiglu_bwd", (16, 16, 16, 16, 16, 1 << 20, 1 << 12, 1 << 12, 1 << 12, 1 << 12,
                            1 << 12, 1 << 12, 0, None), "2\\^31"),
        # keep bits need n_cols % 8 == 0; the LoRA input-gradient kernel d % 32 == 0
        ("rus_dropout_keep_bits", (16, 0, 2, 4, 12, 0.1, 0.1, 16, None), "multiple of 8"),
        ("rus_lora_bwd_x", (16, 16, 4, 64, 64, 16, 16, 16, 16, 16, 48, 16, 16, 16, 48, None,
                            None, 0.0, 0.0, 16, 1 << 20, 16, 64, None), "d % 32"),
        # LoRA workspace smaller than the split reduction needs; no counters
        ("rus_lora_down_fwd", (16, 100, 64, 64, 16, 16, 16, 16, 16, None, None, 0.0, 0.0, 16, 10,
                               16, 64, None), "workspace holds"),
        ("rus_lora_bwd_w", (16, 64, None, None, 0.0, 0.0, 16, 16, 16, 16, 16, 16, 100, 64, 64, 64,
                            16, 16, 16, 16, 16, 16, 1 << 20, None, 0, None), "counters"),
        # attention: head_dim other than 128, GQA ratio not integral, misaligned output
        ("rus_attn_varlen_fwd", (16, 16, 16, 16, 1, 32, 2, 12, 2, 64, 0.1, 16, 16, None),
         "head_dim"),
        ("rus_attn_varlen_fwd", (16, 16, 16, 16, 1, 32, 2, 12, 5, 128, 0.1, 16, 16, None),
         "multiple"),
        ("rus_attn_varlen_fwd", (16, 16, 16, 16, 1, 32, 2, 12, 2, 128, 0.1, 18, 16, None),
         "output"),
        ("rus_attn_varlen_bwd", (16, 16, 16, 16, 16, 16, 16, 1, 32, 2, 12, 2, 128, 0.1, 16, 16,
                                 16, None, None, 0, None), "misaligned"),
        ("rus_attn_varlen_bwd", (16, 16, 16, 16, 16, 16, 16, 1, 32, 2, 12, 2, 128, 0.1, 16, 16,
                                 16, 16, 16, 3, None), "counters"),
        # split-partial norm backward: n_parts out of range, width not a multiple of 8
        ("rus_rmsnorm_bwd_parts", (16, 0, 16, 16, 0, 16, None, 16, 4, 64, 64, None), "n_parts"),
        ("rus_rmsnorm_bwd_parts", (16, 65, 16, 16, 0, 16, None, 16, 4, 64, 64, None), "n_parts"),
        # split-K product: K not a multiple of 64, N not a multiple of 8, a split count that does
        # not cut K into 64-wide pieces, a misaligned operand, an unknown B layout
        ("rus_gemm_parts", (16, 96, 16, 96, 1, 4, 8, 96, 16, 1, None), "not a multiple of 64"),
        ("rus_gemm_parts", (16, 64, 16, 16, 1, 4, 12, 64, 16, 1, None), "not a multiple of 8"),
        ("rus_gemm_parts", (16, 128, 16, 16, 1, 4, 16, 128, 16, 3, None), "does not divide"),
        ("rus_gemm_parts", (8, 64, 16, 16, 1, 4, 16, 64, 16, 1, None), "16-byte aligned"),
        ("rus_gemm_parts", (16, 64, 16, 16, 2, 4, 16, 64, 16, 1, None), "bad sizes"),
        ("rus_rmsnorm_bwd_parts", (16, 2, 16, 16, 0, 16, None, 16, 4, 60, 60, None),
         "multiples of 8"),
        # LoRA weight gradients + expansion: width not a multiple of 32, missing dx
        ("rus_lora_bwd_xw", (16, 40, None, None, 0.0, 0.0, 16, 16, 16, 16, 16, 16, 4, 40, 16, 16,
                             16, 16, 16, 16, 16, 16, 16, 16, 40, 16, 4096, 16, 4, None),
         "need d"),
        ("rus_lora_bwd_xw", (16, 64, None, None, 0.0, 0.0, 16, 16, 16, 16, 16, 16, 4, 64, 16, 16,
                             16, 16, 16, 16, 16, 16, 16, None, 64, 16, 8192, 16, 4, None),
         "null pointer"),
        # RoPE backward with d_mid: rank other than 16, a head layout a block cannot hold
        ("rus_qkv_rope_bwd_mid", (16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 8, 16, 16, 4, 2048,
                                  128, 8, 1.0, 1.0, 12, 2, 128, None, None), "rank"),
        ("rus_qkv_rope_bwd_mid", (16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 4, 2304,
                                  128, 8, 1.0, 1.0, 12, 3, 128, None, None), "slots"),
        # the partial-sum variants: a missing partial buffer, a missing workspace
        ("rus_qkv_rope_bwd_mid_parts", (16, None, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16, 16,
                                        4, 2304, 128, 8, 1.0, 1.0, 12, 2, 128, None, None),
         "null pointer"),
        ("rus_attn_varlen_bwd_parts", (16, 16, 16, 16, 16, 16, 16, 1, 32, 2, 12, 2, 128, 0.1, 16,
                                       None, None), "null or misaligned"),
        # LoRA cast: five segments, a null input, an empty segment
        ("rus_lora_cast_t", (16, 2, 5, None, None, 16, None, None), "n_seg"),
        ("rus_lora_cast_t", (None, 2, 1, (ctypes.c_int64 * 1)(4), (ctypes.c_int64 * 1)(4), 16,
                             None, None), "null pointer"),
        ("rus_lora_cast_t", (16, 2, 1, (ctypes.c_int64 * 1)(0), (ctypes.c_int64 * 1)(4), 16,
                             None, None), "segment 0"),
        # AdamW: a missing moment, a misaligned buffer, a beta of 1, a negative size, step 0
        ("rus_adamw_step", (16, 16, 16, None, 5, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, None),
         "null pointer"),
        ("rus_adamw_step", (16, 8, 16, 16, 5, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, None),
         "16-byte aligned"),
        ("rus_adamw_step", (16, 16, 16, 16, 5, 1e-3, 1.0, 0.999, 1e-8, 0.01, 1, None), "betas"),
        ("rus_adamw_step", (16, 16, 16, 16, -1, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, None),
         "bad size"),
        ("rus_adamw_step", (16, 16, 16, 16, 5, 1e-3, 0.9, 0.999, 1e-8, 0.01, 0, None), "step"),
    ],
)
def test_invalid_arguments_are_rejected_on_the_host(name, args, msg):
    # Pointer values here are never dereferenced: validation fails before any launch.
    with pytest.raises(RuntimeError, match=msg):
        _lib.call(name, *args)


def test_multi_dequant_validates_every_job():
    jobs = (_lib.Nf4Job * 2)()
    for j in jobs:
        j.packed = j.absmax = j.absmax2 = j.out_u32 = 16
        j.split_byte_1 = j.split_byte_2 = j.n_bytes = 64
        j.n_absmax, j.n_absmax2 = 4, 1
    jobs[1].n_absmax = 1  # second job's absmax too short for its bytes
    with pytest.raises(RuntimeError, match="absmax has 1 entries"):
        _lib.call("rus_nf4_dequant_multi", jobs, 2, 16, 64, 256, None)


@pytest.mark.parametrize("field,value,msg", [("kind", 3, "kind"), ("n_cols", 4096, "the norm needs"),
                                             ("n_cols", 1500, "the norm needs"),
                                             ("out", None, "null norm operand")])
def test_dequant_with_norm_validates_the_norm_first(field, value, msg):
    # The norm side of the combined launch is checked before any job; nothing is launched.
    jobs = (_lib.Nf4Job * 1)()
    side = _lib.NormSide()
    side.kind, side.w_dtype = _lib.NORM_FWD, 1
    side.n_rows, side.n_cols, side.stride_row, side.eps = 8, 1536, 1536, 1e-6
    side.x = side.weight = side.rstd = side.out = 16
    setattr(side, field, value)
    if field == "n_cols":
        side.stride_row = value
    with pytest.raises(RuntimeError, match=msg):
        _lib.call("rus_nf4_dequant_multi_norm", jobs, 1, 16, 64, 256, side, None, None)


def _rows_args(**kw):
    a = _lib.LoraRows()
    a.x, a.stride_x, a.n_tokens, a.d, a.r = 16, 1536, 8, 1536, 16
    a.a_q = a.a_v = a.mid_q = a.mid_v = 16
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,msg", [({"r": 32}, "rank 32"), ({"d": 1500, "stride_x": 1500},
                                    "multiple of 64"), ({"bits_q": 16}, "both branches"),
                                    ({"p_q": 1.0, "bits_q": 16, "bits_v": 16}, "probabilities"),
                                    ({"x": None}, "null pointer"), ({"x": 8}, "16-byte aligned")])
def test_lora_down_rows_validates(kw, msg):
    with pytest.raises(RuntimeError, match=msg):
        _lib.call("rus_lora_down_rows", _rows_args(**kw), None)


def test_dequant_carried_lora_down_must_read_the_norm_output():
    # The LoRA-down the combined launch carries reads the forward norm's own output rows; it is
    # checked with the norm, before any job, so nothing is launched.
    jobs = (_lib.Nf4Job * 1)()
    side = _lib.NormSide()
    side.kind, side.w_dtype = _lib.NORM_FWD, 1
    side.n_rows, side.n_cols, side.stride_row, side.eps = 8, 1536, 1536, 1e-6
    side.x = side.weight = side.rstd = 16
    side.out = 32
    for kw in ({"x": 48}, {"n_tokens": 9}, {"d": 1024}):
        with pytest.raises(RuntimeError, match="forward norm's output rows"):
            _lib.call("rus_nf4_dequant_multi_norm", jobs, 1, 16, 64, 256, side,
                      _rows_args(**{"x": 32, **kw}), None)
    side.kind = _lib.NORM_BWD
    side.h = 16
    with pytest.raises(RuntimeError, match="forward norm's output rows"):
        _lib.call("rus_nf4_dequant_multi_norm", jobs, 1, 16, 64, 256, side, _rows_args(x=32),
                  None)


def test_lora_workspace_sizes_follow_the_block_decomposition():
    from rus_amd import kernels as K

    # down: d / 128 reduction chunks x ceil(n / 32) token tiles x one 32 x 32 fp32 partial
    assert K.lora_workspace_size(K.LORA_DOWN, 736, 1536, 1, 1, 16) == (12 * 23 * 1024, 23)
    # rank 32 keeps the branches in two accumulators; d = 48 reduces in chunks of 16
    assert K.lora_workspace_size(K.LORA_DOWN, 33, 48, 1, 1, 32) == (3 * 2 * 2048, 2)
    # d_mid: (d_q + d_v) / 128 chunks per tile
    assert K.lora_workspace_size(K.LORA_BWD_X, 736, 1536, 1536, 256, 16) == (14 * 23 * 1024, 23)
    # weight gradients: 64-column blocks over (2 d + d_q + d_v) x 128-token chunks x [r, 64]
    assert K.lora_workspace_size(K.LORA_BWD_W, 736, 1536, 1536, 256, 16) == \
        (6 * 76 * 16 * 64, 76)
    assert K.lora_workspace_size(K.LORA_BWD_W, 0, 1536, 1536, 256, 8) == (76 * 8 * 64, 76)
    with pytest.raises(RuntimeError, match="unknown entry point"):
        K.lora_workspace_size(7, 1, 64, 64, 64, 16)


@pytest.mark.parametrize(
    "name,args,msg",
    [
        # kept logits: null buffer, stride below round_up(n_vocab, 64)
        ("rus_lmhead_ce_fwd_keep", (16, 16, 16, 4, 64, 64, 64, 100, 0, 16, 16, 16, 16, 0, 4, 16,
                                    None, 128, None), "null logits"),
        ("rus_lmhead_ce_fwd_keep", (16, 16, 16, 4, 64, 64, 64, 100, 0, 16, 16, 16, 16, 0, 4, 16,
                                    16, 120, None), "ld_z"),
        ("rus_lmhead_ce_grad_from_logits", (16, 120, 16, 16, 16, 4, 100, 0, None), "ld_g"),
        ("rus_lmhead_ce_grad_from_logits", (16, 128, None, 16, 16, 4, 100, 0, None), "null"),
    ],
)
def test_kept_logit_entry_points_validate_on_the_host(name, args, msg):
    with pytest.raises(RuntimeError, match=msg):
        _lib.call(name, *args)


def test_lm_head_split_count_fills_whole_rounds_of_workgroups():
    from rus_amd import kernels as K

    def abi_ok(k, s):  # the C ABI's rule: n_split = ceil(K / round_up(ceil(K / n_split), 64))
        per = -(-k // s)
        per = -(-per // 64) * 64
        return s == -(-k // per)

    # config 5 (707 tokens): 3 x 6 tiles; 14 splits = 252 blocks, one round on 256 CUs
    assert K.lm_head_split_count(707, 1536, 151936) == 14
    # config 2 (2048 tokens): 8 x 6 tiles; 16 splits = 768 blocks, three full rounds
    assert K.lm_head_split_count(2048, 1536, 151936) == 16
    for n, d, v in [(707, 1536, 151936), (17, 256, 700), (300, 256, 1031), (64, 64, 64)]:
        kp = -(-v // 64) * 64
        s = K.lm_head_split_count(n, d, v)
        assert 1 <= s <= 64 and abi_ok(kp, s)
        for cap in (1, 2, 5):
            c = K.lm_head_split_count(n, d, v, max_split=cap)
            assert c <= cap and abi_ok(kp, c)


def test_lm_head_token_blocks_take_whole_tiles_within_the_logit_budget():
    from rus_amd import kernels as K

    # V = 151936: three 256-token tiles of fp16 logits fit the 256 MiB budget
    assert K.lm_head_block_tokens(151936) == 768
    assert K.lm_head_block_tokens(151936) * 151936 * 2 <= K.LM_BLOCK_BUDGET
    assert K.lm_head_block_tokens(10**9) == 256  # at least one tile
    assert K.lm_head_token_blocks(0, 768) == []
    assert K.lm_head_token_blocks(1, 768) == [(0, 1)]
    assert K.lm_head_token_blocks(5, 768) == [(0, 3), (3, 5)]  # within one tile: two halves
    assert K.lm_head_token_blocks(744, 768) == [(0, 512), (512, 744)]  # never all N at once
    assert K.lm_head_token_blocks(1100, 768) == [(0, 768), (768, 1100)]
    assert K.lm_head_token_blocks(744, 256) == [(0, 256), (256, 512), (512, 744)]
    for n in (2, 5, 255, 256, 257, 707, 1088, 2048, 5000):
        tiles = -(-n // 256)
        for cap in (1, 256, 300, 768, 1792, 10**6):
            blocks = K.lm_head_token_blocks(n, cap)
            # contiguous cover of [0, n), at least two blocks (no block holds every token)
            assert blocks[0][0] == 0 and blocks[-1][1] == n and len(blocks) >= 2
            assert all(a[1] == b[0] and a[0] < a[1] for a, b in zip(blocks, blocks[1:]))
            if tiles == 1:
                continue
            # whole tiles but the last; no more tiles than n needs; fewest blocks within the cap
            max_tiles = max(1, min(cap // 256, tiles - 1))
            assert all((t1 - t0) % 256 == 0 for t0, t1 in blocks[:-1])
            assert all(0 < t1 - t0 <= max_tiles * 256 for t0, t1 in blocks)
            assert sum(-(-(t1 - t0) // 256) for t0, t1 in blocks) == tiles
            assert len(blocks) == -(-tiles // max_tiles)


def test_lm_head_layout_never_holds_a_whole_vocabulary_row_by_default():
    from rus_amd import kernels as K
    from rus_amd import ops

    V = 151936
    for n in (1, 100, 256, 442, 707, 768, 876, 2048, 8192):
        c = ops.lm_head_layout(None, n, V, "cpu")
        assert c % K.LM_TILE == 0 and c < V, (n, c)
        assert ops.lm_head_layout(-1, n, V, "cpu") == c
        assert n * c * 2 <= max(K.LM_CHUNK_BUDGET, n * K.LM_TILE * 2)
    # whole-vocabulary choices split into two chunks of whole tiles
    assert ops.lm_head_layout(None, 64, 4099, "cpu") == 2304
    assert ops.lm_head_layout(None, 64, 200, "cpu") == 256  # one tile: one chunk
    assert ops.lm_head_layout(0, 707, V, "cpu") is None  # the token-blocked head
    assert ops.lm_head_layout(8192, 707, V, "cpu") == 8192
