"""``pick``: the launch configuration the attention path runs, with an explanation.

Same call as the reference's ``pick(op, shape, dtype, arch, override, cache,
profile, explain, **kwargs)`` (``src/stackkernels/_opt/pick.py:18-226``) for the
ops of this path -- ``flash_attn`` / ``flash_attention`` / ``flash_fwd``,
``flash_bwd`` and ``flash_decode``.  The reference resolves a Triton config
(override > user cache > shipped tuned file > class heuristic) that its
attention launchers then mostly ignore.  Here the tiles are compiled into
``libsk_attn.so`` as a gfx950 table, so the answer comes from the library
(``sk_kernel_config``): the kernel the launcher would run, its tile sizes,
wavefronts, ring depth, grid, split count and scratch, and -- on a GPU -- the
LDS, registers and resident workgroups per CU the HIP runtime reports.  An
``override`` is returned as given, as in the reference; for ``flash_decode`` its
``SPLIT_KV`` is the ``num_splits`` the launcher accepts, and the rest of the
answer is worked out for it.

Shapes: ``flash_attn`` / ``flash_bwd`` take q's shape (B, H_q, S_q, D) with
``kv_len`` (S_k, default S_q), ``num_kv_heads`` (default H_q) and
``is_causal`` keywords, or a dict with ``batch``, ``heads``, ``kv_heads``,
``seq_q``, ``seq_k``, ``head_dim``.  ``flash_decode`` takes q's shape
(B, H_q, 1, D) with ``kv_len`` and ``num_kv_heads``; ``kv_len`` is honoured
(the reference's decode seed reads ``shape[2]``, q's length 1, instead).
"""

from __future__ import annotations

import ctypes
from typing import Any

from stackkernels_amd._opt.hardware import DeviceProfile, get_device_profile, mi355x_profile

_FWD_OPS = ("flash_attn", "flash_attention", "flash_fwd")
_BWD_OPS = ("flash_bwd",)
_DECODE_OPS = ("flash_decode",)

_DTYPE_CODES = {"float32": 0, "fp32": 0, "float": 0, "float16": 1, "fp16": 1, "half": 1,
                "bfloat16": 2, "bf16": 2}

# sk_kernel_config ops and cfg slots (include/sk_attn.h).
_OP_FWD, _OP_BWD_DKV, _OP_BWD_DQ, _OP_DECODE, _OP_DECODE_COMBINE = 0, 1, 2, 3, 4
_VARIANT_PAGED, _VARIANT_ROPE, _VARIANT_VARLEN = 1, 2, 4
_SLOTS = ("grid", "threads", "block_m", "block_n", "stages", "head_dim", "splits", "paired",
          "workspace_bytes", "keys_per_split", "lds_bytes", "vgprs", "wg_per_cu", "chunks")


def _dtype_code(dtype: Any) -> int:
    name = str(dtype).replace("torch.", "").lower()
    if name not in _DTYPE_CODES:
        raise ValueError(f"dtype {dtype!r} has no kernel (float32, float16, bfloat16)")
    return _DTYPE_CODES[name]


def _problem(op: str, shape: Any, kwargs: dict[str, Any]) -> dict[str, int]:
    """(B, H_q, H_kv, S_q, S_k, D, causal) of the call pick describes."""
    if isinstance(shape, dict):
        b = int(shape.get("batch", 1))
        hq = int(shape.get("heads", shape.get("num_heads", 1)))
        hkv = int(shape.get("kv_heads", shape.get("num_kv_heads", hq)))
        sq = int(shape.get("seq_q", shape.get("q_len", 1)))
        sk = int(shape.get("seq_k", shape.get("kv_len", sq)))
        d = int(shape.get("head_dim", 64))
    elif isinstance(shape, (list, tuple)) and len(shape) == 4:
        b, hq, sq, d = (int(x) for x in shape)
        hkv = int(kwargs.get("num_kv_heads", kwargs.get("kv_heads", hq)))
        sk = int(kwargs.get("kv_len", kwargs.get("seq_k", sq)))
    else:
        raise ValueError(f"{op}: shape must be q's (B, H_q, S_q, D) or a dict, got {shape!r}")
    if op in _DECODE_OPS:
        sq = 1
    causal = bool(kwargs.get("is_causal", kwargs.get("causal", False))) and op not in _DECODE_OPS
    return dict(B=b, Hq=hq, Hkv=hkv, Sq=sq, Sk=sk, D=d, causal=int(causal))


def kernel_config(op_code: int, dtype: int, prob: dict[str, int], num_splits: int = 0,
                  variant: int = 0, query_device: bool = False) -> dict[str, Any]:
    """One ``sk_kernel_config`` query: the plan's slots and the kernel name."""
    from stackkernels_amd._core.attention import _lib

    lib = _lib.load()
    cfg = (ctypes.c_int64 * 16)()
    name = ctypes.create_string_buffer(256)
    rc = lib.sk_kernel_config(op_code, dtype, prob["B"], prob["Hq"], prob["Hkv"], prob["Sq"],
                              prob["Sk"], prob["D"], prob["causal"], int(num_splits), variant,
                              int(bool(query_device)), cfg, name, 256)
    _lib.check(rc, "sk_kernel_config")
    out = {k: int(cfg[i]) for i, k in enumerate(_SLOTS)}
    out["kernel"] = name.value.decode()
    return out


def _device_query(prof: DeviceProfile) -> bool:
    """Ask the HIP runtime for occupancy only on a gfx950 device in this process."""
    if prof.arch != "gfx950":
        return False
    try:
        import torch

        return bool(torch.cuda.is_available())
    except Exception:
        return False


def _public(k: dict[str, Any]) -> dict[str, Any]:
    """Reference-style keys for one kernel's plan."""
    out = {
        "BLOCK_M": k["block_m"],
        "BLOCK_N": k["block_n"],
        "num_warps": k["threads"] // 64,  # wavefronts per workgroup
        "num_stages": k["stages"],
        "kernel_variant": k["kernel"].split("<")[0],
        "kernel": k["kernel"],
        "grid": k["grid"],
        "head_dim_padded": k["head_dim"],
    }
    for key in ("lds_bytes", "vgprs", "wg_per_cu"):
        if k[key] >= 0:
            out[key] = k[key]
    return out


def pick(
    op: str,
    shape: Any = None,
    dtype: str = "float16",
    arch: str | None = None,
    override: dict[str, Any] | None = None,
    cache: Any = None,
    profile: DeviceProfile | None = None,
    explain: bool = False,
    **kwargs: Any,
) -> dict[str, Any] | tuple[dict[str, Any], str]:
    """Configuration of ``op`` at ``shape``; with ``explain`` also a report.

    ``cache`` is accepted for call compatibility: the kernels' tiles are
    compiled in, so there is no tuned-configuration cache to consult.
    ``kwargs``: ``kv_len``, ``num_kv_heads``, ``is_causal``, ``paged``,
    ``rope`` (decode / forward variants), ``varlen`` (decode with per-row
    cache lengths: its split plan).
    """
    op_name = str(op).strip().lower()
    if op_name not in _FWD_OPS + _BWD_OPS + _DECODE_OPS:
        raise NotImplementedError(
            f"pick: '{op_name}' is not an op of the attention path this package serves "
            f"({', '.join(_FWD_OPS + _BWD_OPS + _DECODE_OPS)})")
    prof = profile or get_device_profile()
    fingerprint = arch or prof.fingerprint()
    code = _dtype_code(dtype)
    prob = _problem(op_name, shape, kwargs)
    variant = ((_VARIANT_PAGED if kwargs.get("paged") else 0) | (_VARIANT_ROPE if kwargs.get("rope") else 0)
               | (_VARIANT_VARLEN if kwargs.get("varlen") else 0))
    query = _device_query(prof)
    splits_req = int((override or {}).get("SPLIT_KV", kwargs.get("num_splits", 0)) or 0)

    kernels: list[dict[str, Any]] = []
    if op_name in _FWD_OPS:
        k = kernel_config(_OP_FWD, code, prob, 0, variant, query)
        kernels.append(k)
        config = _public(k)
        config["paired_causal_blocks"] = bool(k["paired"])
    elif op_name in _BWD_OPS:
        dkv = kernel_config(_OP_BWD_DKV, code, prob, 0, 0, query)
        dq = kernel_config(_OP_BWD_DQ, code, prob, 0, 0, query)
        kernels += [dkv, dq]
        config = _public(dkv)
        config["kernel_variant"] = f"{config['kernel_variant']}+{dq['kernel'].split('<')[0]}"
        config["dq"] = _public(dq)
        config["workspace_bytes"] = dkv["workspace_bytes"]
        # launches of each kernel per call: chunks of (batch, KV head) pairs
        # whose dS tiles fit the workspace (1 for the seven-GEMM backward)
        config["chunks"] = dkv["chunks"]
    else:
        k = kernel_config(_OP_DECODE, code, prob, splits_req, variant, query)
        kernels.append(k)
        config = {"SPLIT_KV": k["splits"], **_public(k), "keys_per_split": k["keys_per_split"],
                  "workspace_bytes": k["workspace_bytes"]}
        if k["splits"] > 1:
            comb = kernel_config(_OP_DECODE_COMBINE, code, prob, splits_req, variant, query)
            kernels.append(comb)
            config["combine"] = _public(comb)

    if override:
        chosen = dict(override)
        source = "user_override"
    else:
        chosen = config
        source = "gfx950 table (libsk_attn.so)"
    if not explain:
        return chosen

    table_prof = prof if prof.is_rocm else mi355x_profile()
    lines = [
        f"=== StackKernels Pick Explanation: '{op_name}' ===",
        f"Decision Source: {source}",
        f"Device Profile: {prof.name} (fingerprint: {fingerprint})",
    ]
    if not prof.is_rocm:
        lines.append(f"  (not a gfx950 device: the entries below are what {table_prof.name} runs)")
    lines += [
        "Hardware Facts:",
        f"  - CU Count: {table_prof.sm_count} (wavefront {table_prof.warp_size} lanes)",
        f"  - Max Threads / CU: {table_prof.max_threads_per_sm}",
        f"  - Registers / CU: {table_prof.max_regs_per_sm}, per lane: {table_prof.max_regs_per_thread}",
        f"  - LDS / CU: {table_prof.max_smem_per_sm} bytes",
        f"  - HBM: {table_prof.peak_bandwidth_gbps} GB/s, bf16 MFMA: "
        f"{(table_prof.peak_tflops or {}).get('bf16')} TFLOP/s (dense)",
        "Problem:",
        f"  - B={prob['B']} H_q={prob['Hq']} H_kv={prob['Hkv']} S_q={prob['Sq']} S_k={prob['Sk']} "
        f"D={prob['D']} causal={bool(prob['causal'])} dtype={dtype}",
        "Kernels & Wave Math:",
    ]
    for k in kernels:
        line = (f"  - {k['kernel']}: grid {k['grid']} workgroups x {k['threads']} threads"
                f" ({k['threads'] // 64} wavefronts)")
        if k["wg_per_cu"] > 0:
            rounds = k["grid"] / (table_prof.sm_count * k["wg_per_cu"])
            line += (f"; {k['wg_per_cu']} resident per CU (LDS {k['lds_bytes']} B, "
                     f"{k['vgprs']} registers per lane) -> {rounds:.2f} rounds over "
                     f"{table_prof.sm_count} CUs")
        else:
            line += f"; {k['grid'] / table_prof.sm_count:.2f} workgroups per CU"
        lines.append(line)
    if op_name in _DECODE_OPS:
        lines.append(f"  - split-KV: {config['SPLIT_KV']} splits of {config['keys_per_split']} keys, "
                     f"{config['workspace_bytes']} bytes of partials")
    if op_name in _BWD_OPS:
        lines.append(f"  - workspace: {config['workspace_bytes']} bytes; each kernel runs "
                     f"{config['chunks']} launch(es), one per chunk of (batch, KV head) pairs "
                     f"whose dS tiles fit (at most 2 GiB of tiles)")
    lines += ["Selected Configuration:", f"  - {chosen}"]
    if override:
        honoured = op_name in _DECODE_OPS and set(override) <= {"SPLIT_KV"}
        lines.append("  (override " + ("applied through num_splits" if honoured else
                     "returned as given: the tiles are compiled in; the launcher runs the "
                     "table's kernels") + ")")
    if op_name in _FWD_OPS and code != 0 and 64 < prob["D"] <= 128:  # not fp32
        lines.append("Rejected Candidates: the other D = 128 forward entry of the table (short "
                     "work: S_q <= 2048, causal S_q <= 4096 or fewer than 2048 blocks of 256 rows, "
                     "unless a query row sees 4096 keys or more on average and the 8-wavefront "
                     "workgroups fill whole rounds of the 256 CUs (a multiple of 256, or 2048 "
                     "or more) "
                     "-> 4 wavefronts, two workgroups per CU, 2-deep ring; else 8 wavefronts, one "
                     "per CU, 4-deep ring)")
    else:
        lines.append("Rejected Candidates: None (one compiled configuration per head dim and "
                     "group size)")
    return chosen, "\n".join(lines)


__all__ = ["pick", "kernel_config"]
