"""Build and load the gfx950 HIP library ``libflaggems_vllm_amd.so`` and the
torch extension ``_fgv_torch.so`` over it.

Both are built in-tree (next to this file) by ``build()``.  ``lib()`` loads
the C-ABI library with ctypes; ``torch_ext()`` imports the extension, whose
C++ functions check arguments and launch the main op and the sibling op
through the same C ABI (and register them as torch.ops.flaggems_vllm ops).
There is no fallback: if either is missing or cannot be loaded, the ops raise.
"""
import ctypes
import glob
import importlib.machinery
import importlib.util
import os
import subprocess
import sysconfig

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG_DIR)  # flaggems-vllm_amd/
_CSRC = os.path.join(_ROOT, "csrc")
_INCLUDE = os.path.join(os.path.dirname(_ROOT), "include")
LIB_PATH = os.path.join(_PKG_DIR, "libflaggems_vllm_amd.so")
EXT_NAME = "_fgv_torch"
EXT_PATH = os.path.join(_PKG_DIR, EXT_NAME + ".so")
EXT_SOURCE = os.path.join(_CSRC, "torch_ops.cpp")

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # RoPE and FP8 parity rely on separately rounded products and sums.
    "-ffp-contract=off",
    # Packed FP32 (v_pk_*_f32) is kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def sources():
    return sorted(glob.glob(os.path.join(_CSRC, "*.hip")))


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{what} failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")


def ext_command(out):
    """g++ line of the torch extension: host C++ against torch's headers and
    libraries and the C-ABI library next to it (found at run time through
    an $ORIGIN rpath)."""
    import torch

    tdir = os.path.dirname(os.path.abspath(torch.__file__))
    tinc, tlib = os.path.join(tdir, "include"), os.path.join(tdir, "lib")
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    return [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-I{tinc}", f"-I{os.path.join(tinc, 'torch', 'csrc', 'api', 'include')}",
        f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include", f"-I{_INCLUDE}",
        EXT_SOURCE, "-o", out,
        f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
        f"-Wl,-rpath,{tlib}",
        f"-L{_PKG_DIR}", "-lflaggems_vllm_amd", "-Wl,-rpath,$ORIGIN",
    ]


def build(verbose=False):
    """Compile every HIP source into LIB_PATH, then the torch extension into
    EXT_PATH (always recompiles both)."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, f"-I{_INCLUDE}", f"-I{_CSRC}", *sources(), "-o", tmp], "hipcc", verbose)
    os.replace(tmp, LIB_PATH)
    tmp = EXT_PATH + ".tmp"
    _run(ext_command(tmp), "g++ (torch extension)", verbose)
    os.replace(tmp, EXT_PATH)
    return LIB_PATH


_ext = None


def torch_ext():
    """The imported torch extension (registers torch.ops.flaggems_vllm's C++
    ops on first import); raises RuntimeError if it is not built."""
    global _ext
    if _ext is not None:
        return _ext
    if not os.path.exists(EXT_PATH):
        raise RuntimeError(
            f"{EXT_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'`. flaggems_vllm has no non-HIP fallback."
        )
    lib()  # the C ABI it links, loaded first from this directory
    loader = importlib.machinery.ExtensionFileLoader(f"flaggems_vllm.{EXT_NAME}", EXT_PATH)
    spec = importlib.util.spec_from_file_location(f"flaggems_vllm.{EXT_NAME}", EXT_PATH, loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    _ext = mod
    return _ext


def raise_status(rc: int, what: str):
    """Raise for a non-zero status of a torch-extension function:
    AssertionError for a failed reference assertion, otherwise as check()."""
    if rc == _ext.ASSERT_FAILED:
        raise AssertionError(f"{what}: {_ext.assert_message()}")
    check(rc, what)


_lib = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def lib():
    """The loaded library; raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` (hipcc, gfx950). flaggems_vllm has no non-HIP fallback."
        )
    L = ctypes.CDLL(LIB_PATH)
    L.fgv_version.restype = ctypes.c_int
    L.fgv_version.argtypes = []
    L.fgv_last_error.restype = ctypes.c_char_p
    L.fgv_last_error.argtypes = []
    L.fgv_qnorm_rope_kv_rope_quant_insert.restype = ctypes.c_int
    L.fgv_qnorm_rope_kv_rope_quant_insert.argtypes = [
        _P, _I64, _I64,  # q, q_stride_token, q_stride_head
        _P, _I64,  # kv, kv_stride_token
        _P, _I64, _I64,  # k_cache, cache_block_stride, num_blocks
        _P, _I64,  # slot_mapping, num_tokens_insert
        _P,  # position_ids
        _P, _I64, _I64,  # cos_sin_cache, cos_sin_stride, max_pos
        _I64, _I64,  # num_tokens, num_heads
        ctypes.c_float, _I64,  # eps, cache_block_size
        _P,  # stream
    ]
    L.fgv_inv_rope_fp8_quant.restype = ctypes.c_int
    L.fgv_inv_rope_fp8_quant.argtypes = [
        _P, _I64, _I64,  # o, o_stride_token, o_stride_head
        _P,  # positions
        _P, _I64, _I64,  # cos_sin_cache, cos_sin_stride, max_pos
        _I64, _I64, _I64,  # num_tokens, n_groups, heads_per_group
        _I64, _I64, _I64,  # nope_dim, rope_dim, quant_group_size
        _P, _I64, _I64,  # fp8_out, fp8_stride_group, fp8_stride_token
        _P, _I64, _I64,  # scale_out, scale_stride_group, scale_stride_k
        _I64, ctypes.c_float, ctypes.c_int,  # padded_tokens, eps, tma_aligned_scales
        _P,  # stream
    ]
    L.fgv_dequantize_and_gather_k_cache.restype = ctypes.c_int
    L.fgv_dequantize_and_gather_k_cache.argtypes = [
        _P, _I64, _I64, _I64,  # out, out_stride_req, out_stride_row, out_rows
        _P, _I64, _I64,  # k_cache, cache_block_stride, num_blocks
        _P, _P,  # seq_lens, gather_lens
        _P, _I64, _I64,  # block_table, block_table_stride, max_blocks_per_seq
        _I64, _I64, _I64,  # num_reqs, block_size, offset
        _I64, _I64, _I64,  # nope_dim, rope_dim, scale_slots
        _P,  # stream
    ]
    L.fgv_fused_q_kv_rmsnorm.restype = ctypes.c_int
    L.fgv_fused_q_kv_rmsnorm.argtypes = [
        _P, _I64, _P, _I64, _P, _I64,  # qr, stride, qr_out, stride, q_weight, q_size
        _P, _I64, _P, _I64, _P, _I64,  # kv, stride, kv_out, stride, kv_weight, kv_size
        _I64, ctypes.c_float, ctypes.c_int,  # num_tokens, eps, weight_is_fp32
        _P,  # stream
    ]
    L.fgv_fused_indexer_q_rope_quant.restype = ctypes.c_int
    L.fgv_fused_indexer_q_rope_quant.argtypes = [
        _P, _I64,  # positions, num_tokens
        _P, _I64, _I64, _I64, _I64,  # index_q, strides, num_heads, head_dim
        _P, _I64, _I64, ctypes.c_int,  # cos_sin, stride, max_pos, is_bf16
        _P, _I64, ctypes.c_int,  # weights, stride, is_fp32
        ctypes.c_float, ctypes.c_float,  # softmax_scale, head_scale
        _P, _I64,  # weights_out, stride
        ctypes.c_int,  # use_fp4
        _P, _I64, _I64,  # q_out, strides
        _P, _I64, _I64,  # scale_out, strides
        _P,  # stream
    ]
    L.fgv_compute_slot_mapping.restype = ctypes.c_int
    L.fgv_compute_slot_mapping.argtypes = [
        _I64, _I64, _P, _I64,  # num_tokens, max_num_tokens, query_start_loc, num_reqs
        _P, ctypes.c_int,  # positions, positions_are_int64
        _P, _I64, _I64,  # block_table, stride, max_blocks_per_req
        _P, _I64,  # slot_mapping, block_size
        _I64, _I64, _I64, _I64,  # cp_world_size, cp_rank, interleave, pad_id
        _P,  # stream
    ]
    L.fgv_sparse_mla_decode_model1.restype = ctypes.c_int
    L.fgv_sparse_mla_decode_model1.argtypes = [
        _P, _I64, _I64, _I64,  # q, strides (batch, seq_q, head)
        _P, _I64, _I64, _I64,  # k_cache, block stride, num_blocks, page_size
        _P, _I64, _I64, _I64, _P,  # indices, strides, topk, topk_length
        _P, _I64, _I64, _I64,  # extra_k_cache, block stride, num_blocks, page_size
        _P, _I64, _I64, _I64, _P,  # extra indices, strides, extra topk, extra lengths
        _P, ctypes.c_float,  # attn_sink, softmax_scale
        _P, _I64, _I64, _I64,  # out, strides
        _P, _I64, _I64,  # lse, strides (batch, head)
        _I64, _I64, _I64,  # batch, seq_q, num_heads
        _P, _I64,  # workspace, workspace_bytes
        _P,  # stream
    ]
    L.fgv_sparse_mla_decode_model1_no_alloc.restype = ctypes.c_int
    L.fgv_sparse_mla_decode_model1_no_alloc.argtypes = L.fgv_sparse_mla_decode_model1.argtypes[:-3] + [_P]
    L.fgv_flash_mla_sparse_fwd.restype = ctypes.c_int
    L.fgv_flash_mla_sparse_fwd.argtypes = [
        _P, _I64, _I64,  # q, strides (token, head)
        _P, _I64, _I64,  # kv, row stride, s_kv
        _P, _I64, _I64,  # indices, token stride, topk
        _P, _P, ctypes.c_float,  # topk_length, attn_sink, sm_scale
        _I64, _I64, _I64,  # s_q, h_q, d_qk
        _P, _I64, _I64,  # out, strides (token, head)
        _P, _I64,  # max_logits, token stride
        _P, _I64,  # lse, token stride
        _P,  # stream
    ]
    L.fgv_sparse_mla_decode_workspace_bytes.restype = ctypes.c_int64
    L.fgv_sparse_mla_decode_workspace_bytes.argtypes = [_I64, _I64, _I64, _I64, _I64, _I64]
    L.fgv_sparse_mla_decode_grid.restype = ctypes.c_int
    L.fgv_sparse_mla_decode_grid.argtypes = [_I64, _I64, _I64, _I64, _I64]
    L.fgv_compute_global_topk_indices_and_lens.restype = ctypes.c_int
    L.fgv_compute_global_topk_indices_and_lens.argtypes = [
        _P, _I64, _I64, _I64, _I64,  # topk_indices, strides, num_tokens, topk
        _P, _P, _I64, _I64, _I64, _I64, _P,  # req, block_table, stride, num_reqs, blocks/req, block_size, valid
        _P, _I64, _I64, _P,  # global_indices, strides, lens
        _P,  # stream
    ]
    L.fgv_top_k_per_row_decode.restype = ctypes.c_int
    L.fgv_top_k_per_row_decode.argtypes = [
        _P, _I64, _I64, _I64, _I64,  # logits, strides, num_rows, width
        _I64, _P,  # next_n, seq_lens
        _P, _I64, _I64, _I64,  # indices, strides, top_k
        _P, _I64,  # workspace, bytes
        _P,  # stream
    ]
    L.fgv_top_k_per_row_prefill.restype = ctypes.c_int
    L.fgv_top_k_per_row_prefill.argtypes = [
        _P, _I64, _I64, _I64, _I64,  # logits, strides, num_rows, width
        _P, _P,  # row_starts, row_ends
        _P, _I64, _I64, _I64,  # indices, strides, top_k
        _P, _I64,  # workspace, bytes
        _P,  # stream
    ]
    L.fgv_top_k_per_row_workspace_bytes.restype = ctypes.c_int64
    L.fgv_top_k_per_row_workspace_bytes.argtypes = [_I64, _I64, _I64]
    L.fgv_fp8_einsum_bhr_hdr.restype = ctypes.c_int
    L.fgv_fp8_einsum_bhr_hdr.argtypes = [_P, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                         _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, ctypes.c_int32, _P]
    L.fgv_fp8_einsum_bhr_hdr_ws.restype = ctypes.c_int
    L.fgv_fp8_einsum_bhr_hdr_ws.argtypes = L.fgv_fp8_einsum_bhr_hdr.argtypes[:-1] + [_P, _I64, _P]
    L.fgv_fp8_einsum_workspace_bytes.restype = ctypes.c_int64
    L.fgv_fp8_einsum_workspace_bytes.argtypes = [_I64, _I64, _I64, _I64]
    L.fgv_combine_topk_swa_width.restype = ctypes.c_int64
    L.fgv_combine_topk_swa_width.argtypes = [_I64, _I64]
    L.fgv_combine_topk_swa_indices.restype = ctypes.c_int
    L.fgv_combine_topk_swa_indices.argtypes = [
        _P, _I64, _I64, _I64, _I64,  # topk_indices, strides, num_tokens, columns
        _P, _P, _P, _I64,  # query_start_loc, seq_lens, gather_lens, num_reqs
        _I64, _I64, _I64, _I64, _I64,  # window, compress_ratio, topk, M, N
        _P, _I64, _I64, _P,  # combined, strides, lens
        _P,  # stream
    ]
    L.fgv_indexer_k_quant_and_cache.restype = ctypes.c_int
    L.fgv_indexer_k_quant_and_cache.argtypes = [
        _P, _I64, ctypes.c_int,  # k, k_stride_token, k_is_fp16
        _I64, _I64, _I64,  # num_tokens, head_dim, quant_block_size
        _P, _I64, _I64, _I64,  # kv_cache, cache_block_stride, num_blocks, block_size
        _P, ctypes.c_int,  # slot_mapping, use_ue8m0
        _P,  # stream
    ]
    L.fgv_fp8_fp4_mqa_logits.restype = ctypes.c_int
    L.fgv_fp8_fp4_mqa_logits.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64,  # q, strides (bytes), q_scale, strides
        _P, _I64, _P, _P, _I64, _I64,  # k, stride (bytes), k_scale, weights, strides
        _P, _P, _P, _I64,  # ks, ke, logits, stride
        _I64, _I64, _I64, _I64, ctypes.c_int,  # M, N, num_heads, head_dim, clean
        _P,  # stream
    ]
    L.fgv_fp8_fp4_paged_mqa_logits.restype = ctypes.c_int
    L.fgv_fp8_fp4_paged_mqa_logits.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64,  # q, strides (bytes), q_scale, strides
        _P, _I64, _I64, _I64, _I64,  # kv_cache, block stride, num_blocks, block_size, head_dim
        _P, _I64, _I64,  # weights, strides
        _P, _I64, _P, _I64, _I64, _I64,  # context_lens, rows per length, block_tables, stride, max blocks, rows per table row
        _P, _I64, _I64, _I64, _I64, ctypes.c_int,  # logits, stride, rows, num_heads, max_model_len, clean
        _P,  # stream
    ]
    L.fgv_cp_gather_indexer_k_quant_cache.restype = ctypes.c_int
    L.fgv_cp_gather_indexer_k_quant_cache.argtypes = [
        _P, _I64, _I64, _I64,  # kv_cache, cache_block_stride, num_blocks, block_size
        _I64, _I64,  # head_dim, quant_block_size
        _P, _I64, _P, _I64,  # k_out, stride, scale_out, stride (bytes)
        _P, _I64, _I64,  # block_table, stride, max_blocks_per_seq
        _P, _I64, _I64,  # cu_seqlen, batch_size, num_tokens
        _P,  # stream
    ]
    _lib = L
    return _lib


def check(rc: int, what: str):
    """Map a C-ABI status to a Python exception."""
    if rc == 0:
        return
    if rc < 0:
        msg = lib().fgv_last_error().decode(errors="replace")
        raise ValueError(f"{what}: {msg} (code {rc})")
    raise RuntimeError(f"{what}: HIP launch failed with hipError_t {rc}")


# Exported symbols that include/flaggems_vllm_amd.h declares.
EXPORTED_SYMBOLS = (
    "fgv_version",
    "fgv_last_error",
    "fgv_qnorm_rope_kv_rope_quant_insert",
    "fgv_inv_rope_fp8_quant",
    "fgv_dequantize_and_gather_k_cache",
    "fgv_fused_q_kv_rmsnorm",
    "fgv_fused_indexer_q_rope_quant",
    "fgv_compute_slot_mapping",
    "fgv_sparse_mla_decode_model1",
    "fgv_sparse_mla_decode_workspace_bytes",
    "fgv_sparse_mla_decode_grid",
    "fgv_compute_global_topk_indices_and_lens",
    "fgv_combine_topk_swa_width",
    "fgv_combine_topk_swa_indices",
    "fgv_top_k_per_row_decode",
    "fgv_top_k_per_row_prefill",
    "fgv_top_k_per_row_workspace_bytes",
    "fgv_fp8_einsum_bhr_hdr",
    "fgv_fp8_einsum_bhr_hdr_ws",
    "fgv_fp8_einsum_workspace_bytes",
    "fgv_sparse_mla_decode_model1_no_alloc",
    "fgv_flash_mla_sparse_fwd",
    "fgv_indexer_k_quant_and_cache",
    "fgv_cp_gather_indexer_k_quant_cache",
    "fgv_fp8_fp4_mqa_logits",
    "fgv_fp8_fp4_paged_mqa_logits",
)
