# SPDX-License-Identifier: Apache-2.0
"""Host integration of the ``kivi_int4`` KV-cache dtype: page budget and shapes.

A vLLM-HUST host allocates KV pages before the plugin sees them, so four
host-side facts must know the KIVI byte layout (``docs/int4-host-integration.md
:20-77`` in the reference, plus the two serve-time fixes of
``docs/serving-verification-20261003.md:31-45``):

1. the CLI literal: ``--kv-cache-dtype kivi_int4`` must pass ``CacheConfig``;
2. the storage dtype (``STR_DTYPE_TO_TORCH_DTYPE["kivi_int4"] = uint8``) and
   "this is a quantized cache";
3. the quant mode and page size: ``KVQuantMode.KIVI_INT4`` and a page of
   ``2 * block_size * num_kv_heads * S`` bytes, ``S = D/2 + 8*D/G``;
4. the cache shape ``(2, num_blocks, block_size, num_kv_heads, S)``, with the
   runner passing ``cache_dtype_str`` to ``get_kv_cache_shape`` and keeping V
   the same shape as K (the two regions must be equal).

The functions below are the one place the page formula lives (it is
``KiviByteCacheLayout``'s), and ``apply_host_edits`` writes the four edits
into a host checkout: the inserted host code imports these helpers, and only
on the ``kivi_int4`` branches, so a host without the plugin installed keeps
working for every other dtype.  Each edit finds its construct structurally,
must match exactly once, and the whole set is verified before any file is
written; ``reverse`` restores each file from the original saved next to it,
after checking that the file still holds exactly what the edit wrote.

    python -m vllm_ascend_quantized_kv_cache.host_integration \\
        --vllm /path/to/vllm-hust --ascend /path/to/vllm-ascend-hust [--check | --reverse]
"""

from __future__ import annotations

import argparse
import os
import re
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

#: environment knob the host reads for the KIVI group size (the plugin reads
#: ``cache_config.kivi_group_size``, default 128; the two must agree)
GROUP_SIZE_ENV = "VLLM_KIVI_GROUP_SIZE"
DTYPE = "kivi_int4"
_ORIG_SUFFIX = ".kivi_int4.orig"


# ---------------------------------------------------------------------------
# the page budget (host-side numbers of KiviByteCacheLayout)
# ---------------------------------------------------------------------------


def kivi_int4_group_size() -> int:
    return int(os.environ.get(GROUP_SIZE_ENV, "128"))


def kivi_int4_bytes_per_token_head(head_size: int, group_size: int | None = None) -> int:
    """``S``: bytes per token per kv head on one side -- int4 codes plus an fp32
    scale and an fp32 minimum per group, spread over the group."""
    g = kivi_int4_group_size() if group_size is None else group_size
    if g <= 0 or g % 8 or head_size % 8 or head_size % g:
        raise ValueError(
            f"kivi_int4 needs group_size divisible by 8 and head_size divisible by 8 and by "
            f"group_size, got head_size={head_size}, group_size={g}."
        )
    return head_size // 2 + 8 * head_size // g


def kivi_int4_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                             head_size: int, group_size: int | None = None) -> tuple[int, ...]:
    """The host's KV tensor: ``(2, NB, Bs, KVH, S)`` uint8, K and V regions equal."""
    s = kivi_int4_bytes_per_token_head(head_size, group_size)
    return (2, num_blocks, block_size, num_kv_heads, s)


def kivi_int4_page_size_bytes(block_size: int, num_kv_heads: int, head_size: int,
                              group_size: int | None = None) -> int:
    """Bytes of one page, both sides (147,456 at Bs = 128, KVH = 8, D = G = 128)."""
    return 2 * block_size * num_kv_heads * kivi_int4_bytes_per_token_head(head_size, group_size)


# ---------------------------------------------------------------------------
# the host edits
# ---------------------------------------------------------------------------

_MOD = "vllm_ascend_quantized_kv_cache.host_integration"
_TAG = "# kivi_int4: vllm-ascend-quantized-kv-cache host edit"


class HostPatchError(RuntimeError):
    """An edit's construct is missing or ambiguous (the host has moved on), or
    a file no longer holds what an earlier apply wrote."""


@dataclass(frozen=True)
class HostEdit:
    tree: str  # "vllm" or "ascend"
    relpath: str
    what: str
    edit: Callable[[str], str]


def _one(pattern: str, text: str, what: str, flags: int = 0) -> re.Match:
    found = list(re.finditer(pattern, text, flags))
    if len(found) != 1:
        raise HostPatchError(
            f"{what}: construct matched {len(found)} times, expected 1 -- re-measure the host "
            "before patching"
        )
    return found[0]


def _indent_of(line: str) -> str:
    return line[: len(line) - len(line.lstrip())]


def _body_start(text: str, def_pattern: str, what: str) -> tuple[int, str]:
    """Offset just after a function's signature (and docstring), and the body indent."""
    m = _one(def_pattern, text, what, re.M)
    pos = m.end()
    rest = text[pos:]
    indent = _indent_of(rest.split("\n", 1)[0]) or _indent_of(m.group(0)) + "    "
    doc = re.match(r"[ \t]*(\"\"\"|''')", rest)
    if doc:
        close = rest.find(doc.group(1), doc.end())
        if close < 0:
            raise HostPatchError(f"{what}: unterminated docstring")
        pos += rest.find("\n", close) + 1
    return pos, indent


def _cache_literal(text: str) -> str:
    m = _one(r"CacheDType\s*=\s*Literal\[(.*?)\]", text, "CacheDType literal", re.S)
    body = m.group(1)
    if f'"{DTYPE}"' in body:
        raise HostPatchError("CacheDType literal: kivi_int4 is already there")
    entries = re.findall(r'^([ \t]*)"[^"]+",?[ \t]*$', body, re.M)
    indent = entries[-1] if entries else "    "
    stripped = body.rstrip()
    sep = "" if stripped.endswith(",") else ","
    new_body = f'{stripped}{sep}\n{indent}"{DTYPE}",  {_TAG}\n'
    return text[: m.start(1)] + new_body + text[m.end(1):]


def _storage_dtype(text: str) -> str:
    m = _one(r"^(STR_DTYPE_TO_TORCH_DTYPE\s*(?::[^=]*)?=\s*\{[ \t]*\n)", text,
             "STR_DTYPE_TO_TORCH_DTYPE", re.M)
    line = f'    "{DTYPE}": torch.uint8,  {_TAG}\n'
    return text[: m.end()] + line + text[m.end():]


def _quantized_kv_cache(text: str) -> str:
    pos, indent = _body_start(
        text, r"^[ \t]*def is_quantized_kv_cache\(\s*(\w+)[^)]*\)[^:]*:[ \t]*\n",
        "is_quantized_kv_cache")
    arg = re.search(r"def is_quantized_kv_cache\(\s*(\w+)", text).group(1)
    block = f'{indent}if {arg} == "{DTYPE}":  {_TAG}\n{indent}    return True\n'
    return text[:pos] + block + text[pos:]


def _quant_mode_member(text: str) -> str:
    m = _one(r"^class KVQuantMode\([^)]*\):[ \t]*\n((?:[ \t]+.*\n|[ \t]*\n)+)", text,
             "KVQuantMode", re.M)
    members = re.findall(r"^([ \t]+)(\w+)\s*=\s*(\d+)", m.group(1), re.M)
    if not members:
        raise HostPatchError("KVQuantMode: no integer members")
    if any(name == "KIVI_INT4" for _, name, _ in members):
        raise HostPatchError("KVQuantMode: KIVI_INT4 is already there")
    indent = members[-1][0]
    value = max(int(v) for _, _, v in members) + 1
    last = list(re.finditer(r"^[ \t]+\w+\s*=\s*\d+.*\n", m.group(1), re.M))[-1]
    at = m.start(1) + last.end()
    line = f"{indent}KIVI_INT4 = {value}  {_TAG}: KIVI group int4 + fp32 scale/min\n"
    return text[:at] + line + text[at:]


def _quant_mode_lookup(text: str) -> str:
    pos, indent = _body_start(text, r"^[ \t]*def get_kv_quant_mode\(\s*(\w+)[^)]*\)[^:]*:[ \t]*\n",
                              "get_kv_quant_mode")
    arg = re.search(r"def get_kv_quant_mode\(\s*(\w+)", text).group(1)
    block = (f'{indent}if {arg} == "{DTYPE}":  {_TAG}\n'
             f"{indent}    return KVQuantMode.KIVI_INT4\n")
    return text[:pos] + block + text[pos:]


def _page_size(text: str) -> str:
    m = _one(r"^([ \t]*)else:[ \t]*\n[ \t]*last_dim = self\.head_size \+ self\.head_size_v\b",
             text, "FullAttentionSpec.real_page_size_bytes", re.M)
    ind = m.group(1)
    block = (
        f"{ind}elif self.kv_quant_mode == KVQuantMode.KIVI_INT4:  {_TAG}\n"
        f"{ind}    # both regions hold S bytes per token and kv head (the plugin's layout)\n"
        f"{ind}    from {_MOD} import kivi_int4_bytes_per_token_head\n\n"
        f"{ind}    last_dim = 2 * kivi_int4_bytes_per_token_head(self.head_size)\n"
    )
    return text[: m.start()] + block + text[m.start():]


def _cache_shape(text: str) -> str:
    m = _one(r"^([ \t]*)return \(2, num_blocks, block_size, num_kv_heads, head_size\)[ \t]*$",
             text, "get_kv_cache_shape", re.M)
    ind = m.group(1)
    block = (
        f'{ind}if cache_dtype_str == "{DTYPE}":  {_TAG}\n'
        f"{ind}    from {_MOD} import kivi_int4_kv_cache_shape\n\n"
        f"{ind}    return kivi_int4_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size)\n"
    )
    return text[: m.start()] + block + text[m.start():]


def _state_bytes(text: str) -> str:
    m = _one(r"^([ \t]*)plane_size_bytes = spec\.num_kv_heads \* spec\.head_size \* "
             r"get_dtype_size\(spec\.dtype\)[ \t]*$", text, "plane_size_bytes", re.M)
    ind = m.group(1)
    block = (
        f'{ind}if getattr(spec.kv_quant_mode, "name", None) == "KIVI_INT4":  {_TAG}\n'
        f"{ind}    from {_MOD} import kivi_int4_bytes_per_token_head\n\n"
        f"{ind}    return replace(spec, num_head_slots=2, state_content_bytes=spec.num_kv_heads\n"
        f"{ind}                   * kivi_int4_bytes_per_token_head(spec.head_size))\n"
    )
    return text[: m.start()] + block + text[m.start():]


def _runner_shape_calls(text: str) -> str:
    calls = list(re.finditer(r"attn_backend\.get_kv_cache_shape\(([^()]*)\)", text))
    todo = [c for c in calls if "cache_dtype_str" not in c.group(1)]
    if not todo:
        raise HostPatchError("model runner: no get_kv_cache_shape call without cache_dtype_str")
    out, last = [], 0
    for c in todo:
        args = c.group(1)
        body = args.rstrip()
        tail = args[len(body):]
        if "\n" in args:
            arg_indent = _indent_of([ln for ln in args.split("\n") if ln.strip()][-1])
            add = (f"{'' if body.endswith(',') else ','}\n{arg_indent}cache_dtype_str="
                   f"self.vllm_config.cache_config.cache_dtype,  {_TAG}")
        else:
            add = f"{'' if body.endswith(',') or not body else ', '}cache_dtype_str=" \
                  "self.vllm_config.cache_config.cache_dtype"
        out.append(text[last:c.start(1)] + body + add + tail)
        last = c.end(1)
    out.append(text[last:])
    return "".join(out)


def _equal_regions(text: str) -> str:
    m = _one(r'^([ \t]*)if hasattr\(current_kv_cache_spec, "head_size_v"\):[ \t]*$', text,
             "head_size_v override", re.M)
    ind = m.group(1)
    new = (
        f'{ind}if (getattr(current_kv_cache_spec, "head_size_v", None) is not None  {_TAG}\n'
        f'{ind}        and self.vllm_config.cache_config.cache_dtype != "{DTYPE}"):'
    )
    return text[: m.start()] + new + text[m.end():]


def host_edits() -> list[HostEdit]:
    """The edits, in the order they are applied."""
    return [
        HostEdit("vllm", "vllm/config/cache.py", "CLI literal", _cache_literal),
        HostEdit("vllm", "vllm/utils/torch_utils.py", "storage dtype", _storage_dtype),
        HostEdit("vllm", "vllm/utils/torch_utils.py", "quantized cache", _quantized_kv_cache),
        HostEdit("vllm", "vllm/v1/kv_cache_interface.py", "quant mode", _quant_mode_member),
        HostEdit("vllm", "vllm/v1/kv_cache_interface.py", "quant mode lookup",
                 _quant_mode_lookup),
        HostEdit("vllm", "vllm/v1/kv_cache_interface.py", "page size", _page_size),
        HostEdit("ascend", "vllm_ascend/attention/attention_v1.py", "cache shape", _cache_shape),
        HostEdit("ascend", "vllm_ascend/attention/attention_v1.py", "state bytes", _state_bytes),
        HostEdit("ascend", "vllm_ascend/worker/model_runner_v1.py", "cache_dtype_str",
                 _runner_shape_calls),
        HostEdit("ascend", "vllm_ascend/worker/model_runner_v1.py", "equal K/V regions",
                 _equal_regions),
    ]


def _patched(files: dict[Path, str], roots: dict[str, Path]) -> dict[Path, str]:
    out = dict(files)
    for e in host_edits():
        path = roots[e.tree] / e.relpath
        try:
            out[path] = e.edit(out[path])
        except HostPatchError as err:
            raise HostPatchError(f"{path}: {err}") from None
    return out


def apply_host_edits(vllm_root: str | Path, ascend_root: str | Path, *, reverse: bool = False,
                     check: bool = False) -> list[Path]:
    """Apply (or with ``reverse`` undo) the edits; returns the files changed.

    ``check`` only verifies that every construct is found exactly once.  No
    file is written unless every edit applies.
    """
    roots = {"vllm": Path(vllm_root), "ascend": Path(ascend_root)}
    paths = sorted({roots[e.tree] / e.relpath for e in host_edits()})
    for p in paths:
        if not p.is_file():
            raise HostPatchError(f"{p} is not a file -- wrong checkout?")
        if "site-packages" in p.resolve().parts or "dist-packages" in p.resolve().parts:
            raise HostPatchError(f"refusing to edit an installed package: {p}")
    if reverse:
        originals = {}
        for p in paths:
            orig = p.with_name(p.name + _ORIG_SUFFIX)
            if not orig.is_file():
                raise HostPatchError(f"{p}: no saved original ({orig.name}); nothing to reverse")
            originals[p] = orig.read_text()
        expect = _patched(originals, roots)
        for p in paths:
            if p.read_text() != expect[p]:
                raise HostPatchError(f"{p} changed since the edits were applied; not reverting")
        for p in paths:
            p.write_text(originals[p])
            p.with_name(p.name + _ORIG_SUFFIX).unlink()
        return paths
    for p in paths:
        if p.with_name(p.name + _ORIG_SUFFIX).exists():
            raise HostPatchError(f"{p}: the edits are already applied (a saved original exists)")
    files = {p: p.read_text() for p in paths}
    new = _patched(files, roots)
    if check:
        return []
    for p in paths:
        p.with_name(p.name + _ORIG_SUFFIX).write_text(files[p])
        p.write_text(new[p])
    return paths


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--vllm", required=True, type=Path, help="vllm-hust checkout")
    ap.add_argument("--ascend", required=True, type=Path, help="vllm-ascend-hust checkout")
    group = ap.add_mutually_exclusive_group()
    group.add_argument("--reverse", action="store_true", help="restore the saved originals")
    group.add_argument("--check", action="store_true", help="verify only; write nothing")
    args = ap.parse_args(argv)
    try:
        changed = apply_host_edits(args.vllm, args.ascend, reverse=args.reverse, check=args.check)
    except HostPatchError as err:
        print(f"FAILED: {err}", file=sys.stderr)
        return 1
    verb = "checked" if args.check else ("reverted" if args.reverse else "patched")
    for p in changed:
        print(f"  {verb} {p}")
    print(f"RESULT: host edits {verb}")
    return 0


if __name__ == "__main__":
    sys.exit(main())


__all__ = [
    "DTYPE",
    "GROUP_SIZE_ENV",
    "HostEdit",
    "HostPatchError",
    "apply_host_edits",
    "host_edits",
    "kivi_int4_bytes_per_token_head",
    "kivi_int4_group_size",
    "kivi_int4_kv_cache_shape",
    "kivi_int4_page_size_bytes",
]
