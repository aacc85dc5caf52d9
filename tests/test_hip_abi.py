"""The C ABI of libdli_hip.so on a machine without a GPU: every symbol declared in
include/dli_hip.h is exported, and calls fail with an error text instead of crashing
(the reference's tests/cpp/test_cuda_aot_kernel.cc:4-12 and test_cuda_runtime.cc:4-11)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import torch  # noqa: F401  (load torch's HIP runtime first)

import dli
from dli import hip

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "dli_hip.h")


def declared_in_header():
    text = open(HEADER, encoding="utf-8").read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dli_hip_\w+)\s*\(", text)))


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", dli.hip_library_path()],
                         capture_output=True, text=True, check=True).stdout
    return sorted({line.split()[-1] for line in out.splitlines() if " T " in line})


def test_every_declared_symbol_is_exported_and_bound():
    declared = declared_in_header()
    assert len(declared) > 30
    assert declared == exported_symbols()
    assert declared == hip.declared_symbols()


def test_library_loads_and_reports_target():
    lib = hip.load()
    assert lib.dli_hip_target_arch() == b"gfx950"


def test_no_device_behaviour():
    lib = hip.load()
    if torch.cuda.is_available():
        assert lib.dli_hip_available() == 1
        return
    assert lib.dli_hip_available() == 0
    assert lib.dli_hip_load_error()  # non-empty reason
    assert lib.dli_hip_free(None) == 0  # cudaFreePointer(nullptr) is a no-op
    p = ctypes.c_void_p()
    assert lib.dli_hip_malloc(16, ctypes.byref(p)) == -2
    assert b"unavailable" in lib.dli_hip_last_error()


def test_embedded_code_objects_are_gfx950_elf_images():
    """dli_hip_code_object hands out the embedded code objects (the images dli_hip_module_load
    takes): AMDGPU ELF files; an unknown name is an error."""
    lib = hip.load()
    image, size = ctypes.c_void_p(), ctypes.c_size_t()
    for name in (b"elementwise", b"decode", b"stack", b"mfma_gemm"):
        assert lib.dli_hip_code_object(name, ctypes.byref(image), ctypes.byref(size)) == 0
        head = ctypes.string_at(image.value, 20)
        assert size.value > 1024 and head[:4] == b"\x7fELF"
        assert int.from_bytes(head[18:20], "little") == 224  # e_machine EM_AMDGPU
    assert lib.dli_hip_code_object(b"nope", ctypes.byref(image), ctypes.byref(size)) == -1
    assert b"no embedded code object named nope" in lib.dli_hip_last_error()


def test_grid_zero_launch_and_empty_work_are_noops():
    lib = hip.load()
    assert lib.dli_hip_launch(None, 0, 1, 1, 64, 1, 1, 0, None, None) == 0
    assert lib.dli_hip_add(hip.BF16, None, None, None, 0, 1, None) == 0
    assert lib.dli_hip_linear(hip.F32, hip.F32, None, None, None, None, 0, 5, 5, None) == 0
    assert lib.dli_hip_attention(hip.F32, None, None, None, None, 0, 2, 2, 1, 1, 8, 1, 1.0, None) == 0


def test_invalid_arguments_are_rejected_with_a_message():
    lib = hip.load()
    assert lib.dli_hip_add(hip.I64, None, None, None, 4, 1, None) == -1
    assert b"unsupported dtype" in lib.dli_hip_last_error()
    assert lib.dli_hip_attention(hip.F32, None, None, None, None, 1, 3, 2, 1, 1, 8, 1, 1.0, None) == -1
    assert b"multiple of kv_heads" in lib.dli_hip_last_error()
    # the [B, S, H, D] output exists only on the flash path (bf16, head_dim 64)
    fake = ctypes.c_void_p(256)  # never dereferenced: rejected before any launch
    assert lib.dli_hip_attention_bshd(hip.F32, fake, fake, fake, fake, 1, 2, 2, 4, 4, 8, 1, 1.0,
                                      None) == -1
    assert b"flash kernel" in lib.dli_hip_last_error()
    assert lib.dli_hip_rotary(hip.F32, None, None, None, None, None, None, 1, 1, 1, 1, 3, 1, 4, 0,
                              None, hip.I64, None) == -1
    assert lib.dli_hip_linear(hip.BF16, hip.F16, None, None, None, None, 1, 1, 1, None) == -1


def test_fused_decode_entry_points_reject_invalid_arguments():
    lib = hip.load()
    # the fused residual + RMSNorm kernel holds rows of up to 1024 columns, the per-row reduce
    # of the large-hidden path rows of up to 4096 (multiples of 8)
    assert lib.dli_hip_linear_residual_norm(None, None, None, None, None, None, None, 2, 64, 64,
                                            1e-6, 1, None, 0, None) == -1
    assert b"norm_weight and xn_out are required" in lib.dli_hip_last_error()
    fake = ctypes.c_void_p(256)  # never dereferenced: the size check comes first
    assert lib.dli_hip_linear_residual_norm(None, None, None, None, fake, None, fake, 2, 5000, 64,
                                            1e-6, 1, None, 0, None) == -1
    assert b"at most 4096" in lib.dli_hip_last_error()
    assert lib.dli_hip_linear_residual_norm(None, None, None, None, fake, None, fake, 2, 2048, 64,
                                            1e-6, 1, None, 0, None) == -1
    assert b"residual and h_out are required" in lib.dli_hip_last_error()
    assert lib.dli_hip_linear_residual_norm(None, None, None, None, fake, None, fake, 65, 2048, 64,
                                            1e-6, 1, None, 0, None) == -1
    assert b"batch rows" in lib.dli_hip_last_error()
    assert lib.dli_hip_linear_residual_norm(None, None, None, None, fake, None, fake, 2, 64, 128,
                                            1e-6, 3, None, 0, None) == -1  # 3 > k / 64
    assert b"splits must be in" in lib.dli_hip_last_error()
    assert lib.dli_hip_linear_residual(None, None, None, None, None, 2, 64, 128, 0, None, 0,
                                       None) == -1
    assert lib.dli_hip_lm_head_argmax(None, None, None, hip.F32, None, 2, 100, 2048, None, 0,
                                      None) == -1
    assert b"hidden_size above 1024" in lib.dli_hip_last_error()
    assert lib.dli_hip_gate_up_silu(None, None, None, None, 0, 32, 64, 1e-6, None) == -1
    assert b"batch rows" in lib.dli_hip_last_error()
    # more than 64 rows take the tiled GEMM, which has no RMSNorm prologue
    assert lib.dli_hip_gate_up_silu(None, fake, None, None, 65, 32, 64, 1e-6, None) == -1
    assert b"at most 64 rows" in lib.dli_hip_last_error()
    assert lib.dli_hip_gate_up_silu(None, None, None, None, 65, 30, 64, 1e-6, None) == -1
    assert b"multiple of 16" in lib.dli_hip_last_error()
    assert lib.dli_hip_linear_residual(None, None, None, None, None, 100, 64, 12, 1, None, 0,
                                       None) == -1
    assert b"multiple of 8" in lib.dli_hip_last_error()
    # prefill q|k|v + RoPE + head layout: shape checks before any pointer is used
    assert lib.dli_hip_qkv_rope_heads(None, None, None, None, None, 16, None, None, None, 0, 5,
                                      64, 2, 1, 64, 0, None) == 0  # no rows: nothing to do
    assert lib.dli_hip_qkv_rope_heads(None, None, None, None, None, 16, None, None, None, 1, 5,
                                      64, 2, 1, 60, 0, None) == -1
    assert b"head_dim must be a multiple of 8" in lib.dli_hip_last_error()
    assert lib.dli_hip_qkv_rope_heads(None, None, None, None, None, 16, None, None, None, 1, 5,
                                      60, 2, 1, 64, 0, None) == -1
    assert b"hidden_size must be a positive multiple of 8" in lib.dli_hip_last_error()
    assert lib.dli_hip_qkv_rope_heads(None, None, None, None, None, 16, None, None, None, 1, 5,
                                      64, 2, 1, 64, 0, None) == -1
    assert b"NULL pointer" in lib.dli_hip_last_error()
    assert lib.dli_hip_qkv_rope_append(None, None, None, None, None, None, 8, None, hip.I64, None,
                                       None, None, None, 64, 1, 2, 64, 2, 1, 16, 1e-6, None) == -1
    assert b"positions" in lib.dli_hip_last_error()
    # hidden above 1024: no RMSNorm prologue, and the parts need a workspace
    assert lib.dli_hip_qkv_rope_append_ws(fake, fake, fake, fake, fake, fake, 8, fake, hip.I64,
                                          fake, fake, fake, fake, 64, 1, 2, 3584, 28, 4, 128,
                                          1e-6, None, 0, None) == -1
    assert b"normalize first" in lib.dli_hip_last_error()
    assert lib.dli_hip_qkv_rope_append_ws(fake, None, fake, fake, fake, fake, 8, fake, hip.I64,
                                          fake, fake, fake, fake, 64, 1, 2, 3584, 28, 4, 128,
                                          1e-6, None, 0, None) == -1
    assert b"workspace too small" in lib.dli_hip_last_error()
    assert lib.dli_hip_qkv_rope_append_workspace(64, 896, 14, 2, 64) == 0  # the fused kernel
    # 64 rows: the tiled GEMM's parts (2 K ranges over 72 column tiles of the 4608 q|k|v rows)
    assert lib.dli_hip_qkv_rope_append_workspace(64, 3584, 28, 4, 128) == 2 * 64 * 4608 * 4
    # 8 rows: two skinny K ranges over 288 row tiles
    assert lib.dli_hip_qkv_rope_append_workspace(8, 3584, 28, 4, 128) == 2 * 8 * 4608 * 4
    # partials [splits, m, n] fp32 (256-byte aligned) + one arrival counter per 16-row tile
    assert lib.dli_hip_splitk_workspace(896, 32, 4) == 4 * 32 * 896 * 4 + 256


def test_noalloc_lm_head_rejects_oversized_calls_before_the_device():
    """The no-alloc lm_head entry point checks the call against its 4 MiB static scratch first."""
    lib = hip.load()
    fake = ctypes.c_void_p(256)  # never dereferenced
    assert lib.dli_hip_lm_head_argmax_norm_noalloc(fake, None, 1e-6, fake, None, hip.F32, fake,
                                                   64, 600000, 64, None) == -1
    assert b"above its 4194304-byte maximum" in lib.dli_hip_last_error()
    assert lib.dli_hip_lm_head_argmax_norm_noalloc(fake, None, 1e-6, fake, None, hip.F32, fake,
                                                   65, 1000, 64, None) == -1
    assert b"batch rows" in lib.dli_hip_last_error()


def test_decoder_stack_rejects_invalid_arguments():
    """dli_hip_decoder_stack checks every argument before it touches the device."""
    lib = hip.load()
    layer = hip.DecoderLayer(*([256] * 10))  # fake, never dereferenced
    fake = ctypes.c_void_p(256)

    def call(layers=ctypes.byref(layer), n=1, positions=fake, pos_dtype=hip.I64, block_size=64,
             batch=32, hidden=896, hq=14, hkv=2, d=64, ffn=4864, splits=4, options=None):
        return lib.dli_hip_decoder_stack(layers, n, fake, fake, positions, pos_dtype, fake, fake,
                                         1024, block_size, 64, batch, hidden, hq, hkv, d, ffn,
                                         1e-6, splits, fake, 1 << 20, None, options, None)

    assert call(n=0) == 0  # no layers: nothing to do
    assert call(layers=None) == -1
    assert call(batch=65) == -1
    assert b"batch must be in [1, 64]" in lib.dli_hip_last_error()
    assert call(hidden=2048) == -1
    assert b"hidden_size" in lib.dli_hip_last_error()
    assert call(d=128) == -1
    assert b"head_dim must be 64" in lib.dli_hip_last_error()
    assert call(block_size=16) == -1
    assert call(hq=14, hkv=4) == -1
    assert b"multiple of kv_heads" in lib.dli_hip_last_error()
    assert call(ffn=100) == -1
    assert call(splits=9) == -1
    assert b"down_splits" in lib.dli_hip_last_error()
    assert call(positions=None) == -1
    assert call(pos_dtype=hip.F32) == -1
    assert b"positions" in lib.dli_hip_last_error()
    missing = hip.DecoderLayer(*([256] * 9 + [0]))  # no block table
    assert call(layers=ctypes.byref(missing)) == -1
    assert b"layer 0 has a NULL pointer" in lib.dli_hip_last_error()
    assert lib.dli_hip_decoder_stack_status(None, None, None) == -1
    # per-call options: the attention split count and the trace buffer travel with the call
    assert call(options=ctypes.byref(hip.StackOptions(33, None, 0))) == -1
    assert b"attention_splits must be in [0, 32]" in lib.dli_hip_last_error()
    assert call(options=ctypes.byref(hip.StackOptions(0, 256, 0))) == -1
    assert b"trace_layers must be positive" in lib.dli_hip_last_error()
    # token ids in place of hidden_in (the embedding gathered by the launch)
    assert lib.dli_hip_decoder_stack(ctypes.byref(layer), 1, None, fake, fake, hip.I64, fake,
                                     fake, 1024, 64, 64, 32, 896, 14, 2, 64, 4864, 1e-6, 3, fake,
                                     1 << 20, None, None, None) == -1
    assert b"hidden_in is NULL" in lib.dli_hip_last_error()
    for dtype, table, vocab, msg in ((hip.F32, 256, 1000, b"token_ids must be int64 or int32"),
                                     (hip.I64, None, 1000, b"embedding table"),
                                     (hip.I32, 258, 1000, b"embedding table"),
                                     (hip.I64, 256, 0, b"vocab > 0")):
        opts = hip.StackOptions(0, None, 0, 256, dtype, table, vocab)
        assert call(options=ctypes.byref(opts)) == -1
        assert msg in lib.dli_hip_last_error()
    assert lib.dli_hip_decoder_stack_workspace(24, 32, 896, 14, 2, 64, 4864, 65, 3, 33) == 0
