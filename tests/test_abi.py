"""The C-ABI library loads and exports exactly what include/mtpk.h declares (no device calls)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mtpk.h"


def _code():
    return re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)


def declared():
    return sorted(set(re.findall(r"\b(mtpk_\w+)\s*\(", _code())))


def declared_arity():
    """Parameter count of every prototype in the header (`(void)` counts as none)."""
    out = {}
    for name, params in re.findall(r"\b(mtpk_\w+)\s*\(([^)]*)\)\s*;", _code()):
        params = " ".join(params.split())
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    import _mtpk

    if not _mtpk.LIB_PATH.exists():
        import __graft_entry__

        __graft_entry__.build()
    return _mtpk.lib()


def test_every_declared_symbol_is_exported_and_bound(lib):
    import _mtpk

    names = declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), f"{name} declared in mtpk.h but not exported"
    assert sorted(_mtpk.EXPORTED) == names, "Python binding and header disagree"


def test_header_library_and_binding_agree(lib):
    """A library or binding left from another revision of the header would pass shifted
    arguments (a count where a pointer is expected): the version and every prototype's
    parameter count must match across the three."""
    import _mtpk

    m = re.search(r"#define\s+MTPK_ABI_VERSION\s+(\d+)", HEADER.read_text())
    assert m, "MTPK_ABI_VERSION missing from mtpk.h"
    assert int(m.group(1)) == _mtpk.ABI_VERSION == lib.mtpk_abi_version()
    arity = declared_arity()
    assert sorted(arity) == declared()
    for name, (_, argtypes) in _mtpk._SIGNATURES.items():
        assert len(argtypes) == arity[name], f"{name}: binding has {len(argtypes)} parameters, mtpk.h {arity[name]}"


def test_host_only_entry_points(lib):
    assert lib.mtpk_status_string(0) == b"success"
    assert b"invalid argument" in lib.mtpk_status_string(-1)
    # work-unit bound: distinct experts + assignments / 16
    assert lib.mtpk_moe_max_units(10, 512) == 10
    assert lib.mtpk_moe_max_units(1920, 512) == 512 + 120
    assert lib.mtpk_moe_max_units(0, 512) == 0
    a = lib.mtpk_moe_workspace_bytes(192, 10, 512, 1024, 4096, 1)
    b = lib.mtpk_moe_workspace_bytes(192, 10, 512, 1024, 4096, 0)
    assert a > 1920 * 4096 * 4 and b > a  # f32 x carries three planes
    assert lib.mtpk_argmax_partials(192, 248320) >= 192
    # bf16 experts: ids + units + n_units + two intermediate planes + f32 y
    w = lib.mtpk_moe_dense_workspace_bytes(48, 10, 512, 1024, 4096)
    assert w >= 480 * 4 + 3 * lib.mtpk_moe_max_units(480, 512) * 4 + 2 * 480 * 1024 * 2 + 480 * 4096 * 4


def test_rejected_arguments_launch_nothing(lib):
    """Argument checks run before any HIP call, so they are exercised without a device."""
    buf0 = (ctypes.c_float * 64)()
    assert lib.mtpk_route_topk(None, 1, 1, 8, 8, 2, None, None, 3, None) == -1
    assert lib.mtpk_dequant_mxfp4(None, None, 1, 33, 0, None, None) == -1
    assert lib.mtpk_greedy_accept(None, 4, None, 3, None, None, None, None, 0, None, 1, 4, 3,
                                  None, None, None, None, None, None, None, None, None, None,
                                  None, None) == -1
    assert lib.mtpk_moe_prep(None, 3, None, 0, 10, 0, 512, None, None, 10, None, None) == -1
    # skinny GEMM: rows over 256, K not a multiple of 256, null pointers
    assert lib.mtpk_gemm_workspace_bytes(257, 64, 256, 0) == 0
    assert lib.mtpk_gemm_bf16(None, 4, 256, None, 64, 0, None, 1, None, 0, None) == -1
    assert lib.mtpk_gemm_bf16(p0 := ctypes.addressof(buf0), 4, 300, p0, 64, 0, p0, 1, None, 0, None) == -1
    assert lib.mtpk_gemm_bf16(p0, 257, 256, p0, 64, 0, p0, 1, None, 0, None) == -1
    # bf16 experts: null weights, H not a multiple of 256, an expert range that is not the
    # local expert count, a workspace that is not 256-byte aligned
    f = 0x1000
    args = lambda **kw: [kw.get("x", f), 4, kw.get("h", 256), kw.get("gu", f), f, 8, 256, f, 2, f, 0,
                         2, 0, kw.get("hi", 8), kw.get("ws", f), 1 << 30, f, None]
    assert lib.mtpk_moe_dense(*args(gu=None)) == -1
    assert lib.mtpk_moe_dense(*args(h=320)) == -1
    assert lib.mtpk_moe_dense(*args(hi=9)) == -1
    assert lib.mtpk_moe_dense(*args(ws=f + 16)) == -1
    # row norm: null input, dim not a multiple of 8, unknown kind
    assert lib.mtpk_rownorm(None, 0, 64, 64, None, 0, None, None, 0, 0, 1e-6, 1.0, None, 0, 0, 0,
                            None, None, None, 0, None, 0, 1, 1, 64, None, 0, 0, 0, None) == -1
    buf = (ctypes.c_float * 256)()
    p = ctypes.addressof(buf)
    assert lib.mtpk_rownorm(p, 0, 60, 60, None, 0, None, p, 0, 0, 1e-6, 1.0, None, 0, 0, 0,
                            None, None, None, 0, p, 0, 1, 1, 60, None, 0, 0, 0, None) == -1
    assert lib.mtpk_rownorm(p, 0, 64, 64, None, 0, None, p, 0, 7, 1e-6, 1.0, None, 0, 0, 0,
                            None, None, None, 0, p, 0, 1, 1, 64, None, 0, 0, 0, None) == -1
    # an output token stride below one token's rows, and the residual form with a gather
    assert lib.mtpk_rownorm(p, 0, 64, 64, None, 0, None, p, 0, 0, 1e-6, 1.0, None, 0, 0, 0,
                            None, None, None, 0, p, 0, 1, 1, 64, None, 0, 0, 56, None) == -1
    assert lib.mtpk_rownorm(p, 0, 64, 64, p, 0, p, p, 0, 0, 1e-6, 1.0, None, 0, 0, 0,
                            None, None, None, 0, p, 0, 1, 1, 64, p, 1, 4, 0, None) == -1
    # rejection sampling: null inputs, then a non-positive temperature with valid-looking
    # pointers (nothing is dereferenced before the checks)
    fake = 0x1000
    assert lib.mtpk_rejection_sample(None, None, 1, 4, 3, 100, None, None, None, 0.7, None, 0,
                                     None, None, None, None, None) == -1
    assert lib.mtpk_rejection_sample(fake, fake, 1, 4, 3, 100, fake, fake, fake, 0.0, fake, 1 << 30,
                                     fake, fake, None, None, None) == -1
    assert lib.mtpk_sample_rows(fake, 1, 4, 100, -1.0, fake, fake, 1 << 30, fake, None) == -1
    # fused sampling-mode acceptance: no active mask, then more lanes than the pack takes
    assert lib.mtpk_rejection_accept(fake, fake, 1, 4, 3, 100, fake, fake, fake, 0.7, fake, 1 << 30,
                                     None, fake, fake, None, 0, 3, fake, fake, None, None, None,
                                     None, None, None, None, None, None, fake, fake, None) == -1
    assert lib.mtpk_rejection_accept(fake, fake, 1, 1025, 3, 100, fake, fake, fake, 0.7, fake,
                                     1 << 40, fake, fake, fake, None, 0, 3, fake, fake, None, None,
                                     None, None, None, None, None, None, None, fake, fake, None) == -1
    assert lib.mtpk_rejection_workspace_bytes(48, 3, 248320) >= 48 * 7 * 61 * 8
    assert lib.mtpk_sample_workspace_bytes(4, 100) == lib.mtpk_rejection_workspace_bytes(4, 0, 100)
    # gated delta rule: null state, unsupported k_dim, t out of range, neither output nor commit
    assert lib.mtpk_delta_rule(None, 4, None, 2, 2, 4, 2, 16, 16, fake, fake, fake, fake, fake,
                               None, fake, None) == -1
    assert lib.mtpk_delta_rule(fake, 4, None, 2, 2, 4, 2, 48, 16, fake, fake, fake, fake, fake,
                               None, fake, None) == -1
    assert lib.mtpk_delta_rule(fake, 4, None, 2, 0, 4, 2, 16, 16, fake, fake, fake, fake, fake,
                               None, fake, None) == -1
    assert lib.mtpk_delta_rule(fake, 4, None, 2, 2, 4, 2, 16, 16, fake, fake, fake, fake, fake,
                               None, None, None) == -1
    assert lib.mtpk_delta_rule(fake, 1, None, 2, 2, 4, 2, 16, 16, fake, fake, fake, fake, fake,
                               None, fake, None) == -1  # 2 rows, 1 slot, no slot map


def test_short_work_list_is_rejected(lib):
    """A work list shorter than the unit bound would drop live assignments: prep, gate_up and
    down refuse it before any launch (fake pointers are never dereferenced)."""
    f = 0x1000
    need = lib.mtpk_moe_max_units(1920, 512)
    assert lib.mtpk_moe_prep(f, 2, f, 0, 1920, 0, 512, f, f, need - 1, f, None) == -1
    assert lib.mtpk_moe_gate_up(f, 1, 192, 4096, f, f, 512, 1024, f, f, f, need - 1, 10, f, 2,
                                1920, None) == -1
    assert lib.mtpk_moe_down(f, 2, 1920, 1024, f, f, 512, 4096, f, f, f, need - 1, f, None) == -1


def test_scale_scan_and_slot_arguments_checked(lib):
    f = 0x1000
    assert lib.mtpk_scale_scan(None, f, 16, f, None) == -1
    assert lib.mtpk_scale_scan(f, f, -1, f, None) == -1
    # DeltaNet prep / conv commit need a positive slot count
    assert lib.mtpk_conv_commit(f, 1, f, 0, f, 300, f, 5, 300, 3, 4, None) == -1
    assert lib.mtpk_deltanet_prep(f, 1, 1000, f, f, 0, f, f, f, 2, 4, 2, 16, 4, 16, 4, 1e-6, 0.25,
                                  f, f, f, f, f, None) == -1


def test_moe_layer_supported_mirrors_the_layer_checks(lib):
    """`mtpk_moe_layer_supported` (what `mxfp4_gemv.layer_fits` asks before choosing the fused
    layer) accepts the real layer and refuses each operand outside `mtpk_moe_layer`'s contract;
    `mtpk_moe_layer` refuses the same calls before any launch. Fake pointers are never read. At
    <= 32 rows the co-launched GEMM tiles are 4-wave whatever the CU count, so the verdicts do
    not depend on a device being present."""
    f = 0x10000

    def args(**kw):
        a = dict(h=f, tokens=32, hidden=4096, rg=f, rows=513, sgu=f, sd=f, si=1024, gu=f, gus=f,
                 dn=f, dns=f, local=512, inter=1024, k=10, lo=0, hi=512)
        a.update(kw)
        return [a["h"], a["tokens"], a["hidden"], a["rg"], a["rows"], a["sgu"], a["sd"], a["si"],
                a["gu"], a["gus"], a["dn"], a["dns"], a["local"], a["inter"], a["k"], a["lo"], a["hi"]]

    assert lib.mtpk_moe_layer_supported(*args()) == 1
    assert lib.mtpk_moe_layer_supported(*args(tokens=1)) == 1
    bad = [
        dict(tokens=257),              # over 256 rows
        dict(k=33),                    # top_k over MAX_TOP_K
        dict(rows=5, local=4, hi=4, k=5),   # top_k over the router's experts
        dict(rows=1026, local=1025, hi=1025),  # over MTPK_MAX_ROUTER_EXPERTS
        dict(hidden=4000),             # hidden not a multiple of 256
        dict(si=1000),                 # shared width not a multiple of 256
        dict(h=f + 8),                 # misaligned activations
        dict(gu=f + 4),                # misaligned expert payload
        dict(lo=1),                    # expert range not the local count
        dict(dns=None),                # null scale
        dict(hidden=262144, si=4096),  # shared gate/up bytes past 32-bit offsets
    ]
    ws = f
    for b in bad:
        a = args(**b)
        assert lib.mtpk_moe_layer_supported(*a) == 0, b
        assert lib.mtpk_moe_layer(*a, None, None, ws, 1 << 40, f, None) == -1, b


def test_layer_fits_refuses_without_a_device_call():
    """The Python gate (`layer_fits`) refuses shapes the fused layer does not take, so
    `Model.moe` runs the separate ops instead of raising: here on CPU tensors, which only the
    shape / dtype / alignment checks look at."""
    import mxfp4_gemv
    import torch

    h = torch.zeros(4, 256, dtype=torch.bfloat16)
    ex = {"gate_up": torch.zeros(8, 64, 128, dtype=torch.uint8),
          "gate_up_scale": torch.zeros(8, 64, 8, dtype=torch.uint8),
          "down": torch.zeros(8, 256, 16, dtype=torch.uint8),
          "down_scale": torch.zeros(8, 256, 1, dtype=torch.uint8)}
    rg = torch.zeros(9, 256, dtype=torch.bfloat16)
    sgu = torch.zeros(512, 256, dtype=torch.bfloat16)
    sd = torch.zeros(256, 256, dtype=torch.bfloat16)
    assert mxfp4_gemv.layer_fits(h, rg, sgu, sd, ex, 2, (0, 8))
    assert not mxfp4_gemv.layer_fits(h, rg, sgu, sd, ex, 9, (0, 8))         # top_k > experts
    assert not mxfp4_gemv.layer_fits(h.float(), rg, sgu, sd, ex, 2, (0, 8))  # fp32 rows
    assert not mxfp4_gemv.layer_fits(torch.zeros(300, 256, dtype=torch.bfloat16), rg, sgu, sd, ex, 2, (0, 8))
    assert not mxfp4_gemv.layer_fits(h[:, :128], rg[:, :128], sgu[:, :128], sd[:128], ex, 2, (0, 8))
    assert not mxfp4_gemv.layer_fits(h, rg, sgu, sd, ex, 2, (1, 9))        # range past the router
    assert not mxfp4_gemv.layer_fits(h, rg, sgu, sd, {k: v for k, v in ex.items() if k != "down_scale"},
                                     2, (0, 8))
