"""ctypes binding of libseedvr2_hip.so (the C ABI in include/seedvr2_hip.h).

Thin plumbing for tests, the smoke check and the benchmark: device memory and
streams come from PyTorch, every computation runs in the HIP library.  Loading
fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libseedvr2_hip.so"

SV2_OK = 0
SV2_EINVAL = -1
SV2_EUNSUPPORTED = -2
SV2_EDEVICE = -100

F32, F16, BF16 = 0, 1, 2
ROPE_REFERENCE, ROPE_ABSOLUTE, ROPE_NONE = 0, 1, 2
VERIFY_NONE, VERIFY_IF_PRESENT, VERIFY_STRICT = 0, 1, 2
STAGE_TEXT_PREPARE, STAGE_WINDOWS, STAGE_TEXT_REDUCE, STAGE_ALL = 1, 2, 4, 7

# Exported symbols declared in include/seedvr2_hip.h.
EXPORTS = [
    "sv2_window_plan",
    "sv2_window_index_map",
    "sv2_rope_table_floats",
    "sv2_rope_table_build",
    "sv2_rope_positions_needed",
    "sv2_window_attention_workspace",
    "sv2_window_attention",
    "sv2_window_attention_stages",
    "sv2_window_attention_no_alloc",
    "sv2_qk_prologue",
    "sv2_rmsnorm_ada",
    "sv2_ada_residual",
    "sv2_swiglu",
    "sv2_block_config_default",
    "sv2_block_load",
    "sv2_block_create",
    "sv2_block_get_config",
    "sv2_block_set_runtime_shape",
    "sv2_block_workspace_size",
    "sv2_block_forward",
    "sv2_block_window_rows",
    "sv2_block_last_forward_merged",
    "sv2_sha256",
    "sv2_sha256_file",
    "sv2_verify_checksums",
    "sv2_verify_checksums_strict",
    "sv2_verify_model_set",
    "sv2_block_forward_host",
    "sv2_block_destroy",
    "sv2_block_set_debug",
    "sv2_dit_input_load",
    "sv2_dit_input_create",
    "sv2_dit_input_get_config",
    "sv2_dit_input_workspace_size",
    "sv2_dit_input_forward",
    "sv2_dit_input_destroy",
    "sv2_dit_output_load",
    "sv2_dit_output_create",
    "sv2_dit_output_get_config",
    "sv2_dit_output_workspace_size",
    "sv2_dit_output_forward",
    "sv2_dit_output_destroy",
    "sv2_dit_load",
    "sv2_dit_load_ex",
    "sv2_dit_create",
    "sv2_dit_get_config",
    "sv2_dit_workspace_size",
    "sv2_dit_forward",
    "sv2_dit_destroy",
    "sv2_inner_product_f16",
    "sv2_inner_product_f16_few_workspace",
    "sv2_inner_product_f16_few",
    "sv2_inner_product_f32",
    "sv2_euler_timesteps",
    "sv2_condition_ratio",
    "sv2_make_condition",
    "sv2_make_dit_input",
    "sv2_cfg_workspace_size",
    "sv2_apply_cfg",
    "sv2_euler_step",
    "sv2_euler_endpoint",
    "sv2_last_error",
    "sv2_version",
]


class WindowRule(ctypes.Structure):
    _fields_ = [
        ("frames", ctypes.c_int),
        ("height", ctypes.c_int),
        ("width", ctypes.c_int),
        ("shifted", ctypes.c_int),
        ("wt", ctypes.c_int),
        ("wh", ctypes.c_int),
        ("ww", ctypes.c_int),
    ]


class Window(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("t0", "t1", "h0", "h1", "w0", "w1")]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("rule", WindowRule),
        ("heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("text_len", ctypes.c_int),
        ("eps", ctypes.c_float),
        ("qk_norm", ctypes.c_int),
        ("rope_mode", ctypes.c_int),
        ("rope_table", ctypes.c_void_p),
        ("rope_npos", ctypes.c_int),
        ("vid_qkv", ctypes.c_void_p),
        ("txt_qkv", ctypes.c_void_p),
        ("qkv_dtype", ctypes.c_int),
        ("gamma_q_vid", ctypes.c_void_p),
        ("gamma_k_vid", ctypes.c_void_p),
        ("gamma_q_txt", ctypes.c_void_p),
        ("gamma_k_txt", ctypes.c_void_p),
        ("vid_out", ctypes.c_void_p),
        ("txt_out", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("debug_pre", ctypes.c_void_p),
        ("exact", ctypes.c_int),
    ]


class BlockConfig(ctypes.Structure):
    _fields_ = [
        ("block_index", ctypes.c_int),
        ("shared_weights", ctypes.c_int),
        ("last_layer", ctypes.c_int),
        ("shifted_window", ctypes.c_int),
        ("dim", ctypes.c_int),
        ("heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("mlp_hidden", ctypes.c_int),
        ("norm_eps", ctypes.c_float),
        ("window_t", ctypes.c_int),
        ("window_h", ctypes.c_int),
        ("window_w", ctypes.c_int),
        ("rope_mode", ctypes.c_int),
        ("qk_norm", ctypes.c_int),
        ("fused_gemm", ctypes.c_int),
    ]


# Branch weights in the exporter's order (ada vectors first).
BRANCH_FIELDS = ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate",
                 "w_qkv", "w_proj", "b_proj", "norm_q", "norm_k", "w_gate", "w_in", "w_out")


class BlockBranch(ctypes.Structure):
    _fields_ = [
        ("ada", ctypes.c_void_p * 6),
        ("w_qkv", ctypes.c_void_p),
        ("w_proj", ctypes.c_void_p),
        ("b_proj", ctypes.c_void_p),
        ("norm_q", ctypes.c_void_p),
        ("norm_k", ctypes.c_void_p),
        ("w_gate", ctypes.c_void_p),
        ("w_in", ctypes.c_void_p),
        ("w_out", ctypes.c_void_p),
    ]


BLOCK_DEBUG_FIELDS = ("qkv_vid", "qkv_txt", "attention_vid", "attention_txt", "projected_vid", "projected_txt",
                      "output_vid", "output_txt", "norm_q_vid", "norm_q_txt", "norm_k_vid", "norm_k_txt",
                      "attention_q", "attention_k", "attention_v", "attention_output")


class BlockDebug(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in BLOCK_DEBUG_FIELDS]


class DitInputConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "video_channels", "text_channels", "sinusoidal_dim",
                                            "embedding_dim")]


INPUT_FIELDS = ("w_vid", "b_vid", "w_txt", "b_txt", "w_time_in", "b_time_in", "w_time_hid", "b_time_hid",
                "w_time_out", "b_time_out")


class DitInputWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in INPUT_FIELDS]


class DitOutputConfig(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int), ("output_channels", ctypes.c_int), ("norm_eps", ctypes.c_float)]


OUTPUT_FIELDS = ("norm_weight", "shift", "scale", "w_proj", "b_proj")


class DitOutputWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in OUTPUT_FIELDS]


_lib = None


def load() -> ctypes.CDLL:
    """Loads the HIP library; raises if it is missing (no fallback exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
            "(the HIP path has no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, ip, i = ctypes.c_void_p, ctypes.c_int, ctypes.c_int
    lib.sv2_window_plan.argtypes = [ctypes.POINTER(WindowRule), ctypes.POINTER(Window), i]
    lib.sv2_window_plan.restype = i
    lib.sv2_window_index_map.argtypes = [ctypes.POINTER(WindowRule), vp, vp]
    lib.sv2_window_index_map.restype = i
    lib.sv2_rope_table_floats.argtypes = [i]
    lib.sv2_rope_table_floats.restype = ctypes.c_size_t
    lib.sv2_rope_table_build.argtypes = [i, vp, ctypes.c_float, i, vp]
    lib.sv2_rope_table_build.restype = i
    lib.sv2_rope_positions_needed.argtypes = [ctypes.POINTER(WindowRule), i, i]
    lib.sv2_rope_positions_needed.restype = i
    lib.sv2_window_attention_workspace.argtypes = [ctypes.POINTER(AttnArgs)]
    lib.sv2_window_attention_workspace.restype = ctypes.c_int64
    lib.sv2_window_attention.argtypes = [ctypes.POINTER(AttnArgs), vp]
    lib.sv2_window_attention.restype = i
    lib.sv2_window_attention_stages.argtypes = [ctypes.POINTER(AttnArgs), i, vp]
    lib.sv2_window_attention_stages.restype = i
    lib.sv2_window_attention_no_alloc.argtypes = [ctypes.POINTER(AttnArgs), vp]
    lib.sv2_window_attention_no_alloc.restype = i
    lib.sv2_qk_prologue.argtypes = [ctypes.POINTER(AttnArgs), vp, vp, vp, vp]
    lib.sv2_qk_prologue.restype = i
    lib.sv2_rmsnorm_ada.argtypes = [vp, vp, i, i, i, ctypes.c_float, vp, vp, vp, i, i, vp]
    lib.sv2_rmsnorm_ada.restype = i
    lib.sv2_ada_residual.argtypes = [vp, vp, i, i, i, vp, vp, i, i, vp]
    lib.sv2_ada_residual.restype = i
    lib.sv2_swiglu.argtypes = [vp, vp, i, ctypes.c_int64, vp]
    lib.sv2_swiglu.restype = i
    cfgp = ctypes.POINTER(BlockConfig)
    brp = ctypes.POINTER(BlockBranch)
    lib.sv2_block_config_default.argtypes = [cfgp]
    lib.sv2_block_config_default.restype = None
    lib.sv2_block_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i, ctypes.POINTER(vp)]
    lib.sv2_block_load.restype = i
    lib.sv2_block_create.argtypes = [cfgp, brp, brp, vp, i, i, ctypes.POINTER(vp)]
    lib.sv2_block_create.restype = i
    lib.sv2_block_get_config.argtypes = [vp, cfgp]
    lib.sv2_block_get_config.restype = i
    lib.sv2_block_set_runtime_shape.argtypes = [vp, i, i, i]
    lib.sv2_block_set_runtime_shape.restype = i
    lib.sv2_block_workspace_size.argtypes = [vp, i]
    lib.sv2_block_workspace_size.restype = ctypes.c_int64
    lib.sv2_block_forward.argtypes = [vp, vp, vp, i, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.sv2_block_forward.restype = i
    lib.sv2_sha256.argtypes = [vp, ctypes.c_size_t, vp]
    lib.sv2_sha256.restype = i
    lib.sv2_sha256_file.argtypes = [ctypes.c_char_p, vp]
    lib.sv2_sha256_file.restype = i
    lib.sv2_verify_checksums.argtypes = [ctypes.c_char_p, i]
    lib.sv2_verify_checksums.restype = i
    lib.sv2_verify_checksums_strict.argtypes = [ctypes.c_char_p, i]
    lib.sv2_verify_checksums_strict.restype = i
    lib.sv2_verify_model_set.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i]
    lib.sv2_verify_model_set.restype = i
    lib.sv2_block_window_rows.argtypes = [vp, i]
    lib.sv2_block_window_rows.restype = ctypes.c_int64
    lib.sv2_block_last_forward_merged.argtypes = [vp]
    lib.sv2_block_last_forward_merged.restype = i
    lib.sv2_block_forward_host.argtypes = [vp, vp, vp, i, vp, vp, vp, vp]
    lib.sv2_block_forward_host.restype = i
    lib.sv2_block_set_debug.argtypes = [vp, ctypes.POINTER(BlockDebug)]
    lib.sv2_block_set_debug.restype = i
    lib.sv2_block_destroy.argtypes = [vp]
    lib.sv2_block_destroy.restype = None
    c_f = ctypes.c_float
    lib.sv2_dit_input_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i, ctypes.POINTER(vp)]
    lib.sv2_dit_input_load.restype = i
    lib.sv2_dit_input_create.argtypes = [ctypes.POINTER(DitInputConfig), ctypes.POINTER(DitInputWeights), i, i,
                                         ctypes.POINTER(vp)]
    lib.sv2_dit_input_create.restype = i
    lib.sv2_dit_input_get_config.argtypes = [vp, ctypes.POINTER(DitInputConfig)]
    lib.sv2_dit_input_get_config.restype = i
    lib.sv2_dit_input_workspace_size.argtypes = [vp, i, i, i, i]
    lib.sv2_dit_input_workspace_size.restype = ctypes.c_int64
    lib.sv2_dit_input_forward.argtypes = [vp, vp, i, vp, i, c_f, i, i, i, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.sv2_dit_input_forward.restype = i
    lib.sv2_dit_input_destroy.argtypes = [vp]
    lib.sv2_dit_input_destroy.restype = None
    lib.sv2_dit_output_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i, ctypes.POINTER(vp)]
    lib.sv2_dit_output_load.restype = i
    lib.sv2_dit_output_create.argtypes = [ctypes.POINTER(DitOutputConfig), ctypes.POINTER(DitOutputWeights), i, i,
                                          ctypes.POINTER(vp)]
    lib.sv2_dit_output_create.restype = i
    lib.sv2_dit_output_get_config.argtypes = [vp, ctypes.POINTER(DitOutputConfig)]
    lib.sv2_dit_output_get_config.restype = i
    lib.sv2_dit_output_workspace_size.argtypes = [vp, i, i, i]
    lib.sv2_dit_output_workspace_size.restype = ctypes.c_int64
    lib.sv2_dit_output_forward.argtypes = [vp, vp, vp, i, i, i, vp, i, vp, ctypes.c_size_t, vp]
    lib.sv2_dit_output_forward.restype = i
    lib.sv2_dit_output_destroy.argtypes = [vp]
    lib.sv2_dit_output_destroy.restype = None
    lib.sv2_dit_load.argtypes = [ctypes.c_char_p, i, ctypes.POINTER(vp)]
    lib.sv2_dit_load.restype = i
    lib.sv2_dit_load_ex.argtypes = [ctypes.c_char_p, i, i, ctypes.POINTER(vp)]
    lib.sv2_dit_load_ex.restype = i
    lib.sv2_dit_create.argtypes = [vp, ctypes.POINTER(vp), i, vp, ctypes.POINTER(vp)]
    lib.sv2_dit_create.restype = i
    lib.sv2_dit_get_config.argtypes = [vp, ctypes.POINTER(DitInputConfig), ctypes.POINTER(DitOutputConfig),
                                       ctypes.POINTER(i)]
    lib.sv2_dit_get_config.restype = i
    lib.sv2_dit_workspace_size.argtypes = [vp, i, i, i, i]
    lib.sv2_dit_workspace_size.restype = ctypes.c_int64
    lib.sv2_dit_forward.argtypes = [vp, vp, vp, i, c_f, i, i, i, vp, vp, ctypes.c_size_t, vp]
    lib.sv2_dit_forward.restype = i
    lib.sv2_dit_destroy.argtypes = [vp]
    lib.sv2_dit_destroy.restype = None
    lib.sv2_inner_product_f16.argtypes = [vp, vp, vp, vp, i, i, i, i, vp, vp, vp, vp]
    lib.sv2_inner_product_f16.restype = i
    lib.sv2_inner_product_f16_few_workspace.argtypes = [i, i, i, i]
    lib.sv2_inner_product_f16_few_workspace.restype = ctypes.c_int64
    lib.sv2_inner_product_f16_few.argtypes = [vp, vp, vp, vp, i, i, i, i, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.sv2_inner_product_f16_few.restype = i
    lib.sv2_inner_product_f32.argtypes = [vp, vp, vp, vp, i, i, i, vp]
    lib.sv2_inner_product_f32.restype = i
    i64 = ctypes.c_int64
    lib.sv2_euler_timesteps.argtypes = [i, vp]
    lib.sv2_euler_timesteps.restype = i
    lib.sv2_condition_ratio.argtypes = [c_f, i, i, i]
    lib.sv2_condition_ratio.restype = c_f
    lib.sv2_make_condition.argtypes = [vp, vp, vp, i64, c_f, vp]
    lib.sv2_make_condition.restype = i
    lib.sv2_make_dit_input.argtypes = [vp, vp, vp, i64, i, vp]
    lib.sv2_make_dit_input.restype = i
    lib.sv2_cfg_workspace_size.argtypes = [i64]
    lib.sv2_cfg_workspace_size.restype = i64
    lib.sv2_apply_cfg.argtypes = [vp, vp, vp, i64, c_f, c_f, vp, ctypes.c_size_t, vp]
    lib.sv2_apply_cfg.restype = i
    lib.sv2_euler_step.argtypes = [vp, vp, vp, i64, c_f, c_f, vp]
    lib.sv2_euler_step.restype = i
    lib.sv2_euler_endpoint.argtypes = [vp, vp, vp, i64, c_f, vp]
    lib.sv2_euler_endpoint.restype = i
    lib.sv2_last_error.argtypes = []
    lib.sv2_last_error.restype = ctypes.c_char_p
    lib.sv2_version.argtypes = []
    lib.sv2_version.restype = ctypes.c_char_p
    _lib = lib
    return lib


class Sv2Error(RuntimeError):
    def __init__(self, code: int, what: str):
        msg = load().sv2_last_error().decode()
        super().__init__(f"{what} failed ({code}): {msg}")
        self.code = code


def check(code: int, what: str) -> int:
    if code < 0:
        raise Sv2Error(code, what)
    return code


def rule(frames, height, width, shifted=False, wt=0, wh=0, ww=0) -> WindowRule:
    return WindowRule(frames, height, width, int(bool(shifted)), wt, wh, ww)


def window_plan(r: WindowRule) -> list[tuple[int, int, int, int, int, int]]:
    lib = load()
    n = check(lib.sv2_window_plan(ctypes.byref(r), None, 0), "sv2_window_plan")
    arr = (Window * max(n, 1))()
    check(lib.sv2_window_plan(ctypes.byref(r), arr, n), "sv2_window_plan")
    return [(w.t0, w.t1, w.h0, w.h1, w.w0, w.w1) for w in arr[:n]]


def rope_positions_needed(r: WindowRule, text_len: int, mode: int) -> int:
    return check(load().sv2_rope_positions_needed(ctypes.byref(r), text_len, mode),
                 "sv2_rope_positions_needed")


def rope_table(mode: int, freqs, theta: float, npos: int) -> np.ndarray:
    lib = load()
    n = lib.sv2_rope_table_floats(npos)
    out = np.zeros(n, dtype=np.float32)
    fr = None
    if freqs is not None:
        fr = np.ascontiguousarray(freqs, dtype=np.float32)
    check(lib.sv2_rope_table_build(mode, fr.ctypes.data if fr is not None else None,
                                   ctypes.c_float(theta), npos, out.ctypes.data),
          "sv2_rope_table_build")
    return out


def torch_dtype_code(t) -> int:
    import torch
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[t.dtype]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class WindowAttention:
    """Owns the device-side constants (rope table, workspace) of one attention
    configuration and launches sv2_window_attention on torch tensors."""

    def __init__(self, r: WindowRule, heads: int, text_len: int, *, eps=1e-5, qk_norm=True,
                 rope_mode=ROPE_REFERENCE, freqs=None, theta=10000.0, device="cuda", exact=False):
        import torch
        self.exact = bool(exact)
        self.rule = r
        self.heads = heads
        self.text_len = text_len
        self.eps = eps
        self.qk_norm = qk_norm
        self.rope_mode = rope_mode
        self.npos = rope_positions_needed(r, text_len, rope_mode)
        if rope_mode != ROPE_NONE:
            tab = rope_table(rope_mode, freqs, theta, self.npos)
            self.rope = torch.from_numpy(tab).to(device)
        else:
            self.rope = None
        self.plan = window_plan(r)
        self.device = device
        self.workspace = None

    def args(self, vid_qkv, txt_qkv, gammas, vid_out, txt_out, debug_pre=None) -> AttnArgs:
        gq_v, gk_v, gq_t, gk_t = gammas if gammas is not None else (None,) * 4
        a = AttnArgs()
        a.rule = self.rule
        a.heads = self.heads
        a.head_dim = 128
        a.text_len = self.text_len
        a.eps = self.eps
        a.qk_norm = int(bool(self.qk_norm))
        a.rope_mode = self.rope_mode
        a.rope_table = None if self.rope is None else self.rope.data_ptr()
        a.rope_npos = self.npos
        a.vid_qkv = vid_qkv.data_ptr()
        a.txt_qkv = None if txt_qkv is None else txt_qkv.data_ptr()
        a.qkv_dtype = torch_dtype_code(vid_qkv)
        a.gamma_q_vid = None if gq_v is None else gq_v.data_ptr()
        a.gamma_k_vid = None if gk_v is None else gk_v.data_ptr()
        a.gamma_q_txt = None if gq_t is None else gq_t.data_ptr()
        a.gamma_k_txt = None if gk_t is None else gk_t.data_ptr()
        a.vid_out = vid_out.data_ptr()
        a.txt_out = None if txt_out is None else txt_out.data_ptr()
        a.out_dtype = torch_dtype_code(vid_out)
        a.debug_pre = None if debug_pre is None else debug_pre.data_ptr()
        a.exact = int(self.exact)
        return a

    def workspace_bytes(self, a: AttnArgs) -> int:
        return check(load().sv2_window_attention_workspace(ctypes.byref(a)),
                     "sv2_window_attention_workspace")

    def _bind_workspace(self, a: AttnArgs, device) -> None:
        import torch
        need = self.workspace_bytes(a)
        if need > 0 and (self.workspace is None or self.workspace.numel() < need):
            self.workspace = torch.empty(need, dtype=torch.uint8, device=device)
        a.workspace = None if need == 0 else self.workspace.data_ptr()
        a.workspace_bytes = need

    def __call__(self, vid_qkv, txt_qkv, gammas, vid_out, txt_out, debug_pre=None, stream=None, stages=None):
        """All three launches (sv2_window_attention), or the STAGE_* bits of
        `stages` through sv2_window_attention_stages."""
        a = self.args(vid_qkv, txt_qkv, gammas, vid_out, txt_out, debug_pre)
        self._bind_workspace(a, vid_qkv.device)
        if stages is None:
            check(load().sv2_window_attention(ctypes.byref(a), _stream(stream)), "sv2_window_attention")
        else:
            check(load().sv2_window_attention_stages(ctypes.byref(a), int(stages), _stream(stream)),
                  "sv2_window_attention_stages")

    def run_no_alloc(self, vid_qkv, txt_qkv, gammas, vid_out, txt_out, debug_pre=None, stream=None):
        """The same attention through sv2_window_attention_no_alloc (the
        library's static scratch; no workspace)."""
        a = self.args(vid_qkv, txt_qkv, gammas, vid_out, txt_out, debug_pre)
        check(load().sv2_window_attention_no_alloc(ctypes.byref(a), _stream(stream)),
              "sv2_window_attention_no_alloc")

    def prologue(self, vid_qkv, txt_qkv, gammas, q_out, k_out, v_out, stream=None):
        a = self.args(vid_qkv, txt_qkv, gammas, q_out, None)
        self._bind_workspace(a, vid_qkv.device)
        check(load().sv2_qk_prologue(ctypes.byref(a), _ptr(q_out), _ptr(k_out), _ptr(v_out),
                                     _stream(stream)), "sv2_qk_prologue")


def window_index_map(r: WindowRule, out, stream=None):
    check(load().sv2_window_index_map(ctypes.byref(r), _ptr(out), _stream(stream)),
          "sv2_window_index_map")


def rmsnorm_ada(x, y, eps, emb=None, shift=None, scale=None, slot_base=0, has_ada=True, stream=None):
    rows, dim = x.shape
    check(load().sv2_rmsnorm_ada(_ptr(x), _ptr(y), torch_dtype_code(x), rows, dim, ctypes.c_float(eps),
                                 _ptr(emb), _ptr(shift), _ptr(scale), slot_base, int(bool(has_ada)),
                                 _stream(stream)), "sv2_rmsnorm_ada")


def ada_residual(x, residual, emb=None, gate=None, slot_base=0, mode=0, stream=None):
    rows, dim = x.shape
    check(load().sv2_ada_residual(_ptr(x), _ptr(residual), torch_dtype_code(x), rows, dim, _ptr(emb),
                                  _ptr(gate), slot_base, mode, _stream(stream)), "sv2_ada_residual")


def swiglu(gate, value, stream=None):
    check(load().sv2_swiglu(_ptr(gate), _ptr(value), torch_dtype_code(gate), gate.numel(),
                            _stream(stream)), "sv2_swiglu")


def block_config(**overrides) -> BlockConfig:
    """The reference defaults (block 0 of SeedVR2-3B) with fields replaced."""
    c = BlockConfig()
    load().sv2_block_config_default(ctypes.byref(c))
    for k, v in overrides.items():
        if not hasattr(c, k):
            raise KeyError(k)
        setattr(c, k, v)
    return c


def _branch_struct(ptrs: dict) -> BlockBranch:
    b = BlockBranch()
    for i, name in enumerate(BRANCH_FIELDS[:6]):
        b.ada[i] = ptrs[name]
    for name in BRANCH_FIELDS[6:]:
        setattr(b, name, ptrs[name])
    return b


class DitBlock:
    """One SeedVR2DiTBlock on the device (sv2_block_* of the C ABI).

    Construct with `DitBlock.load(param, bin, dtype)` (an exported block) or
    `DitBlock.from_host(config, weights, dtype)` (numpy fp32 weights:
    {"vid": {field: array}, "txt": {...}, "freqs": [21]}) or
    `DitBlock.from_device(config, weights, dtype)` (torch device tensors,
    matrices in the compute dtype, vectors fp32; borrowed)."""

    def __init__(self, handle: int, dtype: int, keep=None):
        self._h = ctypes.c_void_p(handle)
        self.dtype = dtype
        self._keep = keep
        self.config = BlockConfig()
        check(load().sv2_block_get_config(self._h, ctypes.byref(self.config)), "sv2_block_get_config")

    @classmethod
    def load(cls, param_path, bin_path, dtype=F32) -> "DitBlock":
        h = ctypes.c_void_p()
        check(load().sv2_block_load(str(param_path).encode(), str(bin_path).encode(), dtype,
                                    ctypes.byref(h)), "sv2_block_load")
        return cls(h.value, dtype)

    @classmethod
    def _create(cls, config, weights, dtype, on_device, ptr_of) -> "DitBlock":
        keep = []

        def branch(d):
            ptrs = {}
            for name in BRANCH_FIELDS:
                arr, p = ptr_of(d[name])
                keep.append(arr)
                ptrs[name] = p
            return _branch_struct(ptrs)

        vb = branch(weights["vid"])
        tb = vb if config.shared_weights else branch(weights["txt"])
        freqs = None
        if weights.get("freqs") is not None:
            freqs = np.ascontiguousarray(np.asarray(weights["freqs"], dtype=np.float32).reshape(-1))
            keep.append(freqs)
        h = ctypes.c_void_p()
        check(load().sv2_block_create(ctypes.byref(config), ctypes.byref(vb), ctypes.byref(tb),
                                      None if freqs is None else freqs.ctypes.data, int(on_device), dtype,
                                      ctypes.byref(h)), "sv2_block_create")
        return cls(h.value, dtype, keep if on_device else None)

    @classmethod
    def from_host(cls, config, weights, dtype=F32) -> "DitBlock":
        def ptr_of(a):
            arr = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
            return arr, arr.ctypes.data
        return cls._create(config, weights, dtype, False, ptr_of)

    @classmethod
    def from_device(cls, config, weights, dtype=F32) -> "DitBlock":
        def ptr_of(t):
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError("device weights must be contiguous device tensors")
            return t, t.data_ptr()
        return cls._create(config, weights, dtype, True, ptr_of)

    def set_runtime_shape(self, frames, height, width):
        check(load().sv2_block_set_runtime_shape(self._h, frames, height, width),
              "sv2_block_set_runtime_shape")
        self.shape = (frames, height, width)

    def workspace_size(self, text_len) -> int:
        return check(load().sv2_block_workspace_size(self._h, text_len), "sv2_block_workspace_size")

    def window_rows(self, text_len) -> int:
        """Rows of the window-sequence order (attention_q/k/v/output captures)."""
        return check(load().sv2_block_window_rows(self._h, text_len), "sv2_block_window_rows")

    def last_forward_merged(self) -> bool:
        """Whether the last forward ran the row-wise steps over the video and
        text rows at once."""
        return bool(check(load().sv2_block_last_forward_merged(self._h), "sv2_block_last_forward_merged"))

    def forward(self, vid, txt, emb, vid_out, txt_out, workspace=None, stream=None):
        """vid [T*H*W, dim], txt [L, dim] (compute dtype), emb [6*dim] fp32."""
        self._check_blobs(vid, txt, emb, vid_out, txt_out)
        text_len = 0 if txt is None else txt.shape[0]
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(load().sv2_block_forward(self._h, _ptr(vid), _ptr(txt), text_len, _ptr(emb), _ptr(vid_out),
                                       _ptr(txt_out), _ptr(workspace), ws_bytes, _stream(stream)),
              "sv2_block_forward")

    def forward_host(self, vid, txt, emb, captures: dict | None = None):
        """The host-buffer forward (sv2_block_forward_host): vid [T*H*W, dim],
        txt [L, dim], emb [6*dim] fp32 host arrays; returns (vid_out, txt_out)
        as fp32 numpy arrays.  captures: {field: fp32 host array} of
        BLOCK_DEBUG_FIELDS to fill during this call."""
        dim = self.config.dim
        vid = np.ascontiguousarray(vid, dtype=np.float32)
        txt = np.ascontiguousarray(np.zeros((0, dim), np.float32) if txt is None else txt, dtype=np.float32)
        emb = np.ascontiguousarray(emb, dtype=np.float32).reshape(-1)
        if vid.ndim != 2 or vid.shape[1] != dim or txt.ndim != 2 or txt.shape[1] != dim or emb.size != 6 * dim:
            raise ValueError("forward_host: vid/txt must be [rows, dim] and emb [6*dim]")
        vo = np.empty_like(vid)
        to = np.empty_like(txt)
        dbg = None
        if captures:
            dbg = BlockDebug()
            for k, a in captures.items():
                if k not in BLOCK_DEBUG_FIELDS:
                    raise KeyError(k)
                if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous):
                    raise ValueError(f"{k}: host captures are contiguous fp32 numpy arrays")
                setattr(dbg, k, a.ctypes.data)
        L = txt.shape[0]
        check(load().sv2_block_forward_host(self._h, vid.ctypes.data, txt.ctypes.data if L else None, L,
                                            emb.ctypes.data, vo.ctypes.data, to.ctypes.data if L else None,
                                            ctypes.byref(dbg) if dbg is not None else None),
              "sv2_block_forward_host")
        return vo, to

    def set_debug(self, captures: dict | None):
        """captures: {field: fp32 contiguous device tensor} for fields of
        BLOCK_DEBUG_FIELDS, or None to stop capturing."""
        if captures is None:
            self._debug = None
            check(load().sv2_block_set_debug(self._h, None), "sv2_block_set_debug")
            return
        d = BlockDebug()
        for k, t in captures.items():
            if k not in BLOCK_DEBUG_FIELDS:
                raise KeyError(k)
            if not (t.is_cuda and t.is_contiguous()) or t.dtype.itemsize != 4 or not t.dtype.is_floating_point:
                raise ValueError(f"{k}: captures are contiguous fp32 device tensors")
            setattr(d, k, t.data_ptr())
        self._debug = captures
        check(load().sv2_block_set_debug(self._h, ctypes.byref(d)), "sv2_block_set_debug")

    def _check_blobs(self, vid, txt, emb, vid_out, txt_out):
        """The blob checks of SeedVR2DiTBlock::forward (seedvr2_dit_block.cpp:
        1119-1138) plus what the C ABI cannot see through plain pointers:
        device, dtype and contiguity of every tensor."""
        import torch
        dim = self.config.dim
        want = torch.float32 if self.dtype == F32 else torch.float16
        shape = getattr(self, "shape", None)

        def ok(t, rows):
            return (t is not None and t.is_cuda and t.is_contiguous() and t.dtype == want and t.dim() == 2
                    and t.shape[1] == dim and (rows is None or t.shape[0] == rows))

        if shape is not None and not ok(vid, shape[0] * shape[1] * shape[2]):
            raise ValueError(f"vid must be a contiguous {want} device tensor [T*H*W={shape}, {dim}]")
        if shape is not None and not ok(vid_out, vid.shape[0]):
            raise ValueError("vid_out must match vid")
        if txt is not None and (not ok(txt, None) or not ok(txt_out, txt.shape[0])):
            raise ValueError(f"txt / txt_out must be contiguous {want} device tensors [L, {dim}]")
        if not (emb.is_cuda and emb.dtype == torch.float32 and emb.is_contiguous() and emb.numel() == 6 * dim):
            raise ValueError(f"emb must be a contiguous fp32 device tensor of {6 * dim} values")

    def close(self):
        if self._h is not None and self._h.value:
            load().sv2_block_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _host_f32(a):
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return arr, arr.ctypes.data


def _dev_ptr(t):
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("device weights must be contiguous device tensors")
    return t, t.data_ptr()


def _need_f32_dev(t, numel, what):
    import torch
    if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float32 and t.numel() == numel):
        raise ValueError(f"{what} must be a contiguous fp32 device tensor of {numel} values")


class _Handle:
    _destroy = None

    def close(self):
        if self._h is not None and self._h.value:
            getattr(load(), self._destroy)(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DitInput(_Handle):
    """The SeedVR2DiTInput head (sv2_dit_input_*)."""
    _destroy = "sv2_dit_input_destroy"

    def __init__(self, handle, dtype, keep=None):
        self._h = ctypes.c_void_p(handle)
        self.dtype = dtype
        self._keep = keep
        self.config = DitInputConfig()
        check(load().sv2_dit_input_get_config(self._h, ctypes.byref(self.config)), "sv2_dit_input_get_config")

    @classmethod
    def load(cls, param_path, bin_path, dtype=F32):
        h = ctypes.c_void_p()
        check(load().sv2_dit_input_load(str(param_path).encode(), str(bin_path).encode(), dtype, ctypes.byref(h)),
              "sv2_dit_input_load")
        return cls(h.value, dtype)

    @classmethod
    def create(cls, weights, dtype=F32, *, on_device=False, video_channels=None, sinusoidal_dim=None):
        keep, ptrs = [], {}
        for k in INPUT_FIELDS:
            arr, p = (_dev_ptr if on_device else _host_f32)(weights[k])
            keep.append(arr)
            ptrs[k] = p
        dim = int(weights["b_vid"].shape[0])
        cfg = DitInputConfig(dim, video_channels or int(weights["w_vid"].shape[1]) // 4,
                             int(weights["w_txt"].shape[1]), sinusoidal_dim or int(weights["w_time_in"].shape[1]),
                             int(weights["b_time_out"].shape[0]))
        w = DitInputWeights(*[ptrs[k] for k in INPUT_FIELDS])
        h = ctypes.c_void_p()
        check(load().sv2_dit_input_create(ctypes.byref(cfg), ctypes.byref(w), int(on_device), dtype, ctypes.byref(h)),
              "sv2_dit_input_create")
        return cls(h.value, dtype, keep if on_device else None)

    def forward(self, video, text, timestep, T, H, W, vid_out, txt_out, emb, *, channel_major=False,
                workspace=None, stream=None):
        """video fp32 [T*H*W, C] (or [C, T, H, W] with channel_major), text fp32
        [L, text_channels]; vid_out / txt_out in the compute dtype, emb fp32."""
        import torch
        c = self.config
        want = torch.float32 if self.dtype == F32 else torch.float16
        _need_f32_dev(video, T * H * W * c.video_channels, "video")
        L = 0 if text is None else text.shape[0]
        if L:
            _need_f32_dev(text, L * c.text_channels, "text")
            if not (txt_out.is_cuda and txt_out.is_contiguous() and txt_out.dtype == want
                    and txt_out.numel() == L * c.dim):
                raise ValueError("txt_out shape/dtype")
        if not (vid_out.is_cuda and vid_out.is_contiguous() and vid_out.dtype == want
                and vid_out.numel() == T * (H // 2) * (W // 2) * c.dim):
            raise ValueError("vid_out shape/dtype")
        _need_f32_dev(emb, c.embedding_dim, "emb")
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(load().sv2_dit_input_forward(self._h, _ptr(video), int(channel_major), _ptr(text), L,
                                           ctypes.c_float(timestep), T, H, W, _ptr(vid_out), _ptr(txt_out if L else None),
                                           _ptr(emb), _ptr(workspace), ws_bytes, _stream(stream)),
              "sv2_dit_input_forward")


class DitOutput(_Handle):
    """The SeedVR2DiTOutput head (sv2_dit_output_*)."""
    _destroy = "sv2_dit_output_destroy"

    def __init__(self, handle, dtype, keep=None):
        self._h = ctypes.c_void_p(handle)
        self.dtype = dtype
        self._keep = keep
        self.config = DitOutputConfig()
        check(load().sv2_dit_output_get_config(self._h, ctypes.byref(self.config)), "sv2_dit_output_get_config")

    @classmethod
    def load(cls, param_path, bin_path, dtype=F32):
        h = ctypes.c_void_p()
        check(load().sv2_dit_output_load(str(param_path).encode(), str(bin_path).encode(), dtype, ctypes.byref(h)),
              "sv2_dit_output_load")
        return cls(h.value, dtype)

    @classmethod
    def create(cls, weights, dtype=F32, *, on_device=False, eps=1e-5):
        keep, ptrs = [], {}
        for k in OUTPUT_FIELDS:
            arr, p = (_dev_ptr if on_device else _host_f32)(weights[k])
            keep.append(arr)
            ptrs[k] = p
        cfg = DitOutputConfig(int(weights["norm_weight"].shape[0]), int(weights["b_proj"].shape[0]) // 4, eps)
        w = DitOutputWeights(*[ptrs[k] for k in OUTPUT_FIELDS])
        h = ctypes.c_void_p()
        check(load().sv2_dit_output_create(ctypes.byref(cfg), ctypes.byref(w), int(on_device), dtype,
                                           ctypes.byref(h)), "sv2_dit_output_create")
        return cls(h.value, dtype, keep if on_device else None)

    def forward(self, vid, emb, T, h, w, output, *, channel_major=False, workspace=None, stream=None):
        import torch
        c = self.config
        want = torch.float32 if self.dtype == F32 else torch.float16
        if not (vid.is_cuda and vid.is_contiguous() and vid.dtype == want and vid.numel() == T * h * w * c.dim):
            raise ValueError("vid shape/dtype")
        _need_f32_dev(emb, 6 * c.dim, "emb")
        _need_f32_dev(output, T * 4 * h * w * c.output_channels, "output")
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(load().sv2_dit_output_forward(self._h, _ptr(vid), _ptr(emb), T, h, w, _ptr(output), int(channel_major),
                                            _ptr(workspace), ws_bytes, _stream(stream)), "sv2_dit_output_forward")


class Dit(_Handle):
    """The whole DiT (sv2_dit_*): input head, blocks, output head."""
    _destroy = "sv2_dit_destroy"

    def __init__(self, handle, dtype, parts=None):
        self._h = ctypes.c_void_p(handle)
        self.dtype = dtype
        self._parts = parts  # borrowed heads and blocks kept alive
        ic, oc, n = DitInputConfig(), DitOutputConfig(), ctypes.c_int()
        check(load().sv2_dit_get_config(self._h, ctypes.byref(ic), ctypes.byref(oc), ctypes.byref(n)),
              "sv2_dit_get_config")
        self.input_config, self.output_config, self.block_count = ic, oc, n.value
        self.video_channels = ic.video_channels
        self.text_channels = ic.text_channels
        self.output_channels = oc.output_channels

    @classmethod
    def load(cls, model_dir, dtype=F32, verify=None):
        """sv2_dit_load (verify None: the manifest checked when present) or
        sv2_dit_load_ex with VERIFY_NONE / VERIFY_IF_PRESENT / VERIFY_STRICT."""
        h = ctypes.c_void_p()
        if verify is None:
            check(load().sv2_dit_load(str(model_dir).encode(), dtype, ctypes.byref(h)), "sv2_dit_load")
        else:
            check(load().sv2_dit_load_ex(str(model_dir).encode(), dtype, verify, ctypes.byref(h)),
                  "sv2_dit_load_ex")
        return cls(h.value, dtype)

    @classmethod
    def create(cls, input_head, blocks, output_head):
        arr = (ctypes.c_void_p * max(len(blocks), 1))(*[b._h.value for b in blocks])
        h = ctypes.c_void_p()
        check(load().sv2_dit_create(input_head._h, arr, len(blocks), output_head._h, ctypes.byref(h)),
              "sv2_dit_create")
        return cls(h.value, input_head.dtype, (input_head, list(blocks), output_head))

    def workspace_size(self, T, H, W, text_len) -> int:
        return check(load().sv2_dit_workspace_size(self._h, T, H, W, text_len), "sv2_dit_workspace_size")

    def forward(self, latent, text, timestep, output, *, workspace=None, stream=None):
        """latent fp32 [C, T, H, W], text fp32 [L, text_channels], output fp32
        [output_channels, T, H, W] (device tensors)."""
        import torch
        C, T, H, W = latent.shape
        for name, t in (("latent", latent), ("output", output)):
            if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float32):
                raise ValueError(f"{name} must be a contiguous fp32 device tensor")
        if tuple(output.shape[1:]) != (T, H, W):
            raise ValueError("output must be [output_channels, T, H, W]")
        if C != self.video_channels or output.shape[0] != self.output_channels:
            raise ValueError("latent / output channel counts differ from the heads")
        L = 0 if text is None else text.shape[0]
        if L and not (text.is_cuda and text.is_contiguous() and text.dtype == torch.float32 and text.dim() == 2
                      and text.shape[1] == self.text_channels):
            raise ValueError("text must be a contiguous fp32 device tensor [L, text_channels]")
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(load().sv2_dit_forward(self._h, _ptr(latent), _ptr(text), L, ctypes.c_float(timestep), T, H, W,
                                     _ptr(output), _ptr(workspace), ws_bytes, _stream(stream)), "sv2_dit_forward")


def euler_timesteps(steps: int) -> np.ndarray:
    """EulerSampler(steps).timesteps() (sampler.cpp:181-187), host."""
    out = np.zeros(max(1, steps), np.float32)
    n = check(load().sv2_euler_timesteps(steps, out.ctypes.data), "sv2_euler_timesteps")
    return out[:n]


def condition_ratio(noise_scale: float, frames: int, height: int, width: int) -> float:
    """The noise ratio of make_condition_latent (engine.cpp:79-92, :110)."""
    return load().sv2_condition_ratio(noise_scale, frames, height, width)


def _latent(t, what):
    import torch
    if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float32):
        raise ValueError(f"{what} must be a contiguous fp32 device tensor")
    return t


class EulerSampler:
    """The Euler v-lerp sampler of the reference (src/model/sampler.h:18-78)
    on device latents: fp32 contiguous tensors, every update enqueued on the
    stream with no host synchronisation.  Shape mismatches raise ValueError
    where the reference returns Status::InvalidArgument."""

    def __init__(self, steps: int):
        self.timesteps = euler_timesteps(steps)
        self._ws = {}

    def _workspace(self, device):
        import torch
        ws = self._ws.get(device)
        if ws is None:
            ws = torch.empty(load().sv2_cfg_workspace_size(0), dtype=torch.uint8, device=device)
            self._ws[device] = ws
        return ws

    @staticmethod
    def _pair(a, b, what):
        _latent(a, what)
        _latent(b, what)
        if a.shape != b.shape:
            raise ValueError(f"{what}: input shapes differ")

    def apply_cfg(self, positive, negative, scale, rescale, output=None, stream=None):
        """EulerSampler::apply_cfg (sampler.cpp:201-236)."""
        import torch
        self._pair(positive, negative, "apply_cfg")
        out = torch.empty_like(positive) if output is None else _latent(output, "apply_cfg output")
        ws = self._workspace(positive.device) if rescale != 0.0 else None
        check(load().sv2_apply_cfg(_ptr(positive), _ptr(negative), _ptr(out), positive.numel(), scale, rescale,
                                   _ptr(ws), 0 if ws is None else ws.numel(), _stream(stream)), "sv2_apply_cfg")
        return out

    def step_to(self, prediction, current, timestep, next_timestep, output=None, stream=None):
        """EulerSampler::step_to (sampler.cpp:239-265)."""
        import torch
        self._pair(prediction, current, "step_to")
        out = torch.empty_like(current) if output is None else _latent(output, "step_to output")
        check(load().sv2_euler_step(_ptr(prediction), _ptr(current), _ptr(out), current.numel(), timestep,
                                    next_timestep, _stream(stream)), "sv2_euler_step")
        return out

    def endpoint(self, prediction, current, timestep, output=None, stream=None):
        """EulerSampler::endpoint (sampler.cpp:267-285)."""
        import torch
        self._pair(prediction, current, "endpoint")
        out = torch.empty_like(current) if output is None else _latent(output, "endpoint output")
        check(load().sv2_euler_endpoint(_ptr(prediction), _ptr(current), _ptr(out), current.numel(), timestep,
                                        _stream(stream)), "sv2_euler_endpoint")
        return out

    @staticmethod
    def make_condition(encoded, noise, ratio, output=None, stream=None):
        """make_condition_latent (engine.cpp:106-122) with the ratio given, as
        make_condition_vulkan takes it (sampler.cpp:314-335)."""
        import torch
        EulerSampler._pair(encoded, noise, "make_condition")
        out = torch.empty_like(encoded) if output is None else _latent(output, "make_condition output")
        check(load().sv2_make_condition(_ptr(encoded), _ptr(noise), _ptr(out), encoded.numel(), ratio,
                                        _stream(stream)), "sv2_make_condition")
        return out

    @staticmethod
    def make_dit_input(latent, condition, channel_major=True, output=None, stream=None):
        """make_dit_input (engine.cpp:125-149): [16, T, H, W] -> [33, T, H, W];
        channel_major=False: [tokens, 16] -> [tokens, 33] (sampler.cpp:337-357)."""
        import torch
        EulerSampler._pair(latent, condition, "make_dit_input")
        if channel_major:
            if latent.dim() < 2 or latent.shape[0] != 16:
                raise ValueError("make_dit_input: channel-major latents are [16, ...]")
            shape, tokens = (33,) + tuple(latent.shape[1:]), latent.numel() // 16
        else:
            if latent.dim() != 2 or latent.shape[1] != 16:
                raise ValueError("make_dit_input: token-major latents are [tokens, 16]")
            shape, tokens = (latent.shape[0], 33), latent.shape[0]
        out = torch.empty(shape, dtype=torch.float32, device=latent.device) if output is None else output
        _latent(out, "make_dit_input output")
        if tuple(out.shape) != shape:
            raise ValueError(f"make_dit_input: output must be {shape}")
        check(load().sv2_make_dit_input(_ptr(latent), _ptr(condition), _ptr(out), tokens,
                                        1 if channel_major else 0, _stream(stream)), "sv2_make_dit_input")
        return out


EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU = 0, 1, 2


def inner_product_f32(x, w, y, bias=None, stream=None):
    """y = float(sum_i double(x_i) double(w_i) + double(bias)) (sv2_inner_product_f32):
    x fp32 [rows, in], w fp32 [out, in], y fp32 [rows, out], bias fp32 [out]."""
    import torch
    rows, k = x.shape
    out = w.shape[0]
    for name, t, shape in (("x", x, (rows, k)), ("w", w, (out, k)), ("y", y, (rows, out))):
        if t.dtype != torch.float32 or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"inner_product_f32: {name} must be a contiguous fp32 {shape}")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != out):
        raise ValueError("inner_product_f32: bias must be fp32 [out]")
    check(load().sv2_inner_product_f32(_ptr(x), _ptr(w), _ptr(bias), _ptr(y), rows, k, out, _stream(stream)),
          "sv2_inner_product_f32")


def inner_product_f16(x, w, y, epilogue=EPI_STORE, w_value=None, bias=None, gate=None, residual=None,
                      stream=None):
    """y = epilogue(x W^T) on the MFMA kernel (sv2_inner_product_f16): x fp16
    [rows, in], w (and w_value) fp16 [out, in], y fp16 [rows, out]; bias and
    gate fp32 [out], residual fp16 [rows, out] (device tensors)."""
    import torch
    rows, k = x.shape
    out = w.shape[0]
    for name, t, shape in (("x", x, (rows, k)), ("w", w, (out, k)), ("y", y, (rows, out))):
        if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float16 and tuple(t.shape) == shape):
            raise ValueError(f"{name} must be a contiguous fp16 device tensor {shape}")
    for name, t, dt, shape in (("w_value", w_value, torch.float16, (out, k)), ("bias", bias, torch.float32, (out,)),
                               ("gate", gate, torch.float32, (out,)),
                               ("residual", residual, torch.float16, (rows, out))):
        if t is not None and not (t.is_cuda and t.is_contiguous() and t.dtype == dt and tuple(t.shape) == shape):
            raise ValueError(f"{name} must be a contiguous {dt} device tensor {shape}")
    check(load().sv2_inner_product_f16(_ptr(x), _ptr(w), _ptr(w_value), _ptr(y), rows, k, out, epilogue,
                                       _ptr(bias), _ptr(gate), _ptr(residual), _stream(stream)),
          "sv2_inner_product_f16")
    return y


def inner_product_f16_few(x, w, y, epilogue=EPI_STORE, w_value=None, bias=None, gate=None, residual=None,
                          workspace=None, stream=None):
    """y = epilogue(x W^T) for 1-64 rows on the weight-streaming kernel
    (sv2_inner_product_f16_few); arguments as inner_product_f16.  `workspace`
    (a device tensor) receives the split partial sums; when None one of the
    size sv2_inner_product_f16_few_workspace asks for is allocated here."""
    import torch
    rows, k = x.shape
    out = w.shape[0]
    for name, t, shape in (("x", x, (rows, k)), ("w", w, (out, k)), ("y", y, (rows, out))):
        if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float16 and tuple(t.shape) == shape):
            raise ValueError(f"{name} must be a contiguous fp16 device tensor {shape}")
    for name, t, dt, shape in (("w_value", w_value, torch.float16, (out, k)), ("bias", bias, torch.float32, (out,)),
                               ("gate", gate, torch.float32, (out,)),
                               ("residual", residual, torch.float16, (rows, out))):
        if t is not None and not (t.is_cuda and t.is_contiguous() and t.dtype == dt and tuple(t.shape) == shape):
            raise ValueError(f"{name} must be a contiguous {dt} device tensor {shape}")
    lib = load()
    need = check(lib.sv2_inner_product_f16_few_workspace(rows, k, out, epilogue),
                 "sv2_inner_product_f16_few_workspace")
    if workspace is None and need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.sv2_inner_product_f16_few(_ptr(x), _ptr(w), _ptr(w_value), _ptr(y), rows, k, out, epilogue,
                                        _ptr(bias), _ptr(gate), _ptr(residual), _ptr(workspace), ws_bytes,
                                        _stream(stream)),
          "sv2_inner_product_f16_few")
    return y



def sha256(data) -> bytes:
    """SHA-256 digest of a bytes-like object (sv2_sha256)."""
    buf = bytes(data)
    out = ctypes.create_string_buffer(32)
    src = ctypes.c_char_p(buf) if buf else None
    check(load().sv2_sha256(src, len(buf), out), "sv2_sha256")
    return out.raw


def sha256_file(path) -> bytes:
    out = ctypes.create_string_buffer(32)
    check(load().sv2_sha256_file(str(path).encode(), out), "sv2_sha256_file")
    return out.raw


def verify_checksums(directory, threads: int = 0) -> int:
    """Checks `directory`/SHA256SUMS; returns the number of files verified (0
    when there is no manifest), raises Sv2Error on a failed check."""
    return check(load().sv2_verify_checksums(str(directory).encode(), threads), "sv2_verify_checksums")


def verify_checksums_strict(directory, threads: int = 0) -> int:
    """verify_checksums, but a directory without SHA256SUMS is an error."""
    return check(load().sv2_verify_checksums_strict(str(directory).encode(), threads),
                 "sv2_verify_checksums_strict")


def verify_model_set(model_root, bundled_embeddings=None, threads: int = 0) -> int:
    """The model-set check of scripts/verify-models.sh for the DiT (strict
    manifest, the 68 DiT files, the default embeddings against the bundled
    copies when a directory of them is given)."""
    b = None if bundled_embeddings is None else str(bundled_embeddings).encode()
    return check(load().sv2_verify_model_set(str(model_root).encode(), b, threads), "sv2_verify_model_set")
