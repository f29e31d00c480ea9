"""Device-side block-FP8 operations on PyTorch-ROCm tensors (thin wrappers over libgk_fp8.so).

These are the fast-path entry points: no host synchronisation (except the
codec and the finite-input check, which read a status word back), caller's
current HIP stream, workspaces from the PyTorch caching allocator.  The
reference-compatible functions (``block_fp8_oracle.reference`` and
``fp8_codec.reencode_e4m3fn_half``) are built on these.

Layouts (row-major): x bf16 [M, K] (unit column stride), weight E4M3 codes
[N, K] contiguous (torch.float8_e4m3fn or uint8), scales fp32
[ceil(N/128), ceil(K/128)] contiguous, bias fp32 [N], output bf16 [M, N].
"""

import ctypes

import torch

from gaudi_kernels import _native as nat

_DEVICE_OK = {}


def require_device(device=None):
    """Return the torch.device to run on; raise if it is not a gfx950 GPU with the library loaded."""
    if not torch.cuda.is_available():
        raise RuntimeError("gaudi_kernels: no GPU visible (the block-FP8 path has no CPU fallback)")
    if device is None or device.type != "cuda":
        device = torch.device("cuda", torch.cuda.current_device())
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _DEVICE_OK:
        lib = nat.load()
        _DEVICE_OK[idx] = lib.gk_device_supported(idx) == nat.GK_SUCCESS
    if not _DEVICE_OK[idx]:
        raise RuntimeError(f"gaudi_kernels: device cuda:{idx} is not a gfx950 GPU")
    return torch.device("cuda", idx)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _u8(t):
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


def plan(m, n, k, flags=0, weight=None):
    """(variant, m_pad, workspace_bytes) that gk_fp8_block_gemm_bf16 uses for these sizes."""
    lib = nat.load()
    variant = ctypes.c_int(0)
    m_pad = ctypes.c_int64(0)
    ws = ctypes.c_size_t(0)
    wp = _ptr(weight) if weight is not None else ctypes.c_void_p(256)
    nat.check("gk_fp8_block_gemm_plan",
              lib.gk_fp8_block_gemm_plan(m, n, k, flags, wp, ctypes.byref(variant), ctypes.byref(m_pad),
                                         ctypes.byref(ws)))
    return variant.value, m_pad.value, ws.value


_WORKSPACES = {}


def workspace(nbytes, device=None):
    """A GEMM workspace of at least `nbytes` for the current stream of `device`.

    Cached per (device, stream) and grown on demand, so that calls ordered on
    one stream reuse it without allocating; GEMMs running on several streams
    at once get one workspace per stream.
    """
    device = require_device(device)
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def make_workspace(m, n, k, *, native_half=False, variant=None, device=None):
    """A new workspace sized for one (m, n, k, flags) plan; for callers that manage their own."""
    _, _, nbytes = plan(m, n, k, _flags(native_half, variant))
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=require_device(device))


def _flags(native_half, variant):
    flags = nat.GK_FLAG_NATIVE_HALF if native_half else 0
    if variant is not None:
        flags |= {"decode": nat.GK_FLAG_FORCE_DECODE, "prefill": nat.GK_FLAG_FORCE_PREFILL,
                  "generic": nat.GK_FLAG_FORCE_GENERIC}[variant]
    return flags


def act_quant(x, *, native_half=False, m_pad=None, decode_layout=False):
    """1x128 activation quantization on the GPU -> group-major (codes uint8 [G, m_pad, 128], sa fp32 [G, m_pad]).

    The layout of the reference's quant op output ({128, R, G} FCD-first, generic_fp8_glue.hpp:84-109).
    decode_layout=True (m_pad 16, 32 or 64 -- by default the decode plan's, 16 * ceil-to-{1,2,4}(M/16)) stores each
    group's codes in the decode fragment order (include/gk_fp8.h, GK_FLAG_DECODE_LAYOUT) for
    block_fp8_gemm_q(..., decode_layout=True).
    """
    device = require_device(x.device)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("expected a 2-D bf16 activation with unit column stride")
    m, k = x.shape
    g = (k + 127) // 128
    m_pad = (16 * decode_tiles(m) if decode_layout else m) if m_pad is None else m_pad
    q = torch.empty((g, m_pad, 128), dtype=torch.uint8, device=device)
    sa = torch.empty((g, m_pad), dtype=torch.float32, device=device)
    flags = (nat.GK_FLAG_NATIVE_HALF if native_half else 0) | (nat.GK_FLAG_DECODE_LAYOUT if decode_layout else 0)
    lib = nat.load()
    nat.check("gk_fp8_act_quant_bf16",
              lib.gk_fp8_act_quant_bf16(_ptr(x), m, k, x.stride(0), _ptr(q), _ptr(sa), m_pad, flags,
                                        _stream(device)))
    return q, sa


def decode_tiles(m):
    """16-token column tiles of the decode variant for M <= 64 tokens (its m_pad is 16 times this)."""
    return 1 if m <= 16 else 2 if m <= 32 else 4


def decode_layout_to_standard(q):
    """View helper: codes in the decode fragment layout [G, m_pad, 128] -> the standard [G, m_pad, 128] order."""
    g, m_pad = q.shape[0], q.shape[1]
    # block (group, token tile t), piece (h, l) = bytes [32 (l // 16) + 16 h, +16) of row 16 t + l % 16
    # -> [G, t, h, quad, row, 16]
    return q.reshape(g, m_pad // 16, 2, 4, 16, 16).permute(0, 1, 4, 3, 2, 5).reshape(g, m_pad, 128)


class PackedWeight:
    """E4M3 weight codes [n, k] in the fragment-packed device layout of gk_fp8_pack_weight.

    The load-time packing step that fp8_codec.py:19 leaves to the loader.  Pass it wherever a
    block-FP8 GEMM takes a weight; results are bit-identical to those on the row-major codes.
    """

    def __init__(self, data, n, k):
        self.data, self.n, self.k = data, n, k

    @property
    def shape(self):
        return (self.n, self.k)

    @property
    def device(self):
        return self.data.device


def packed_weight_bytes(n, k):
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check("gk_fp8_packed_weight_bytes", lib.gk_fp8_packed_weight_bytes(n, k, ctypes.byref(nbytes)))
    return nbytes.value


def pack_weight(weight):
    """Row-major E4M3 codes [N, K] (K % 128 == 0) on the GPU -> PackedWeight (asynchronous)."""
    device = require_device(weight.device)
    if weight.dtype not in (torch.float8_e4m3fn, torch.uint8) or weight.ndim != 2 or not weight.is_contiguous():
        raise ValueError("expected a contiguous 2-D E4M3 weight [N, K]")
    n, k = weight.shape
    data = torch.empty(packed_weight_bytes(n, k), dtype=torch.uint8, device=device)
    lib = nat.load()
    nat.check("gk_fp8_pack_weight",
              lib.gk_fp8_pack_weight(_ptr(_u8(weight)), n, k, _ptr(data), data.numel(), _stream(device)))
    return PackedWeight(data, n, k)


class PackedExperts:
    """Expert weights [E, n, k] in the panel-major packed order (pack_experts) for moe_block_fp8."""

    def __init__(self, data, e, n, k):
        self.data, self.e, self.n, self.k = data, e, n, k

    @property
    def shape(self):
        return (self.e, self.n, self.k)

    @property
    def device(self):
        return self.data.device


def pack_experts(weights):
    """Row-major E4M3 expert codes [E, N, K] (K % 128 == 0) on the GPU -> PackedExperts (asynchronous):
    gk_fp8_pack_experts, expert e at byte e * packed_weight_bytes(N, K), each 256-row panel's blocks of one
    128-K group side by side."""
    device = require_device(weights.device)
    if weights.dtype not in (torch.float8_e4m3fn, torch.uint8) or weights.ndim != 3 or not weights.is_contiguous():
        raise ValueError("expected contiguous E4M3 expert weights [E, N, K]")
    e, n, k = weights.shape
    data = torch.empty(e * packed_weight_bytes(n, k), dtype=torch.uint8, device=device)
    nat.check("gk_fp8_pack_experts",
              nat.load().gk_fp8_pack_experts(_ptr(_u8(weights)), e, n, k, _ptr(data), data.numel(), _stream(device)))
    return PackedExperts(data, e, n, k)


def _weight_args(weight):
    """(uint8 tensor passed as w, n, k, extra flags) for a row-major or packed weight."""
    if isinstance(weight, PackedWeight):
        return weight.data, weight.n, weight.k, nat.GK_FLAG_WEIGHT_PACKED
    return _u8(weight), weight.shape[0], weight.shape[1], 0


def _check_gemm_operands(weight, scales, bias, device):
    if isinstance(weight, PackedWeight):
        if weight.data.dtype != torch.uint8 or weight.data.numel() < packed_weight_bytes(weight.n, weight.k):
            raise ValueError("PackedWeight data is not a pack_weight output")
    elif weight.dtype not in (torch.float8_e4m3fn, torch.uint8) or weight.ndim != 2 or not weight.is_contiguous():
        raise ValueError("expected a contiguous 2-D E4M3 weight [N, K]")
    if scales.dtype != torch.float32 or scales.ndim != 2 or not scales.is_contiguous():
        raise ValueError("expected contiguous fp32 block scales [ceil(N/128), ceil(K/128)]")
    if weight.device != device or scales.device != device or (bias is not None and bias.device != device):
        raise ValueError("all operands must be on the same GPU")
    if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous() or bias.numel() != weight.shape[0]):
        raise ValueError("expected a contiguous fp32 bias with N elements")


def block_fp8_gemm(x, weight, scales, bias=None, *, native_half=False, variant=None, out=None, workspace=None):
    """y = block-FP8 W8A8 linear of bf16 x [M, K] with E4M3 weight [N, K] -> bf16 [M, N] (asynchronous).

    weight: row-major codes or a PackedWeight (pack_weight).
    variant: None (dispatch by M), "decode", "prefill" or "generic" (not for packed weights).
    workspace: optional 256-byte aligned uint8 device tensor of at least plan(...)[2] bytes
    (make_workspace); calls that share one workspace must be ordered on one stream.  Default: the
    cached per-stream workspace().
    """
    device = require_device(x.device)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("expected a 2-D bf16 activation with unit column stride")
    _check_gemm_operands(weight, scales, bias, device)
    m, k = x.shape
    w8, n, kw, wflag = _weight_args(weight)
    if kw != k:
        raise ValueError("activation and weight K differ")
    flags = _flags(native_half, variant) | wflag
    _, _, ws_bytes = plan(m, n, k, flags, w8)
    ws = _checked_workspace(workspace, ws_bytes, device)
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    elif out.dtype != torch.bfloat16 or out.shape != (m, n) or out.stride(1) != 1 or out.device != device:
        raise ValueError("out must be bf16 [M, N] with unit column stride on the same GPU")
    lib = nat.load()
    nat.check("gk_fp8_block_gemm_bf16",
              lib.gk_fp8_block_gemm_bf16(_ptr(x), m, k, x.stride(0), _ptr(w8), n, _ptr(scales), scales.shape[0],
                                         scales.shape[1], _ptr(bias), _ptr(out), out.stride(0), flags,
                                         _ptr(ws), ws.numel(), _stream(device)))
    return out


def _checked_workspace(ws, nbytes, device):
    if ws is None:
        return workspace(nbytes, device)
    if ws.dtype != torch.uint8 or ws.device != device or ws.numel() < nbytes or ws.data_ptr() % 256:
        raise ValueError(f"workspace must be a 256-byte aligned uint8 tensor of >= {nbytes} bytes on {device}")
    return ws


def block_fp8_gemm_q(q, sa, m, weight, scales, bias=None, *, native_half=False, variant=None, out=None,
                     decode_layout=False):
    """GEMM on activations already quantized by act_quant(m_pad=plan(...)[1]) (group-major q, sa).

    decode_layout: q comes from act_quant(..., decode_layout=True); the plan must be the decode variant.
    """
    device = require_device(q.device)
    _check_gemm_operands(weight, scales, bias, device)
    w8, n, k, wflag = _weight_args(weight)
    flags = _flags(native_half, variant) | (nat.GK_FLAG_DECODE_LAYOUT if decode_layout else 0) | wflag
    g = (k + 127) // 128
    if q.shape != (g, q.shape[1], 128) or sa.shape != (g, q.shape[1]) or not (q.is_contiguous() and sa.is_contiguous()):
        raise ValueError("expected group-major q [G, m_pad, 128] and sa [G, m_pad] from act_quant")
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    lib = nat.load()
    nat.check("gk_fp8_block_gemm_q_bf16",
              lib.gk_fp8_block_gemm_q_bf16(_ptr(q), _ptr(sa), m, q.shape[1], k, _ptr(w8), n, _ptr(scales),
                                           scales.shape[0], scales.shape[1], _ptr(bias), _ptr(out), out.stride(0),
                                           flags, _stream(device)))
    return out


def _status_workspace(device):
    return torch.empty(256, dtype=torch.uint8, device=device)


def codec_ocp_to_half(codes, scales):
    """GPU forward codec on device tensors -> (half codes uint8, 2*scales, rounded) or GkError."""
    device = require_device(codes.device)
    src = _u8(codes)
    dst = torch.empty_like(src)
    s_out = torch.empty_like(scales)
    ws = _status_workspace(device)
    rounded = ctypes.c_int64(0)
    lib = nat.load()
    nat.check("gk_fp8_codec_ocp_to_half",
              lib.gk_fp8_codec_ocp_to_half(_ptr(src), _ptr(dst), src.numel(), _ptr(scales), _ptr(s_out),
                                           scales.numel(), ctypes.byref(rounded), _ptr(ws), ws.numel(),
                                           _stream(device)))
    return dst, s_out, rounded.value


def codec_half_to_ocp(codes, scales):
    """GPU inverse codec on device tensors -> (OCP codes uint8, scales/2) or GkError."""
    device = require_device(codes.device)
    src = _u8(codes)
    dst = torch.empty_like(src)
    s_out = torch.empty_like(scales)
    ws = _status_workspace(device)
    lib = nat.load()
    nat.check("gk_fp8_codec_half_to_ocp",
              lib.gk_fp8_codec_half_to_ocp(_ptr(src), _ptr(dst), src.numel(), _ptr(scales), _ptr(s_out),
                                           scales.numel(), _ptr(ws), ws.numel(), _stream(device)))
    return dst, s_out


def inputs_finite(x, weight, scales):
    """True iff x is finite, weight holds no OCP NaN code and scales are finite and >= 0 (GPU check)."""
    device = require_device(x.device)
    ws = _status_workspace(device)
    w8 = _u8(weight)
    lib = nat.load()
    st = lib.gk_fp8_check_inputs(_ptr(x), x.shape[0], x.shape[1], x.stride(0), _ptr(w8), w8.shape[0],
                                 _ptr(scales), scales.numel(), _ptr(ws), ws.numel(), _stream(device))
    if st == nat.GK_NONFINITE_INPUT:
        return False
    nat.check("gk_fp8_check_inputs", st)
    return True


def _check_gate_up(gate_up, device):
    if gate_up.dtype != torch.bfloat16 or gate_up.ndim != 2 or gate_up.stride(1) != 1 or gate_up.shape[1] % 2:
        raise ValueError("expected a 2-D bf16 gate_up [rows, 2*width] with unit column stride")
    if gate_up.device != device:
        raise ValueError("gate_up must be on the GPU")
    return gate_up.shape[0], gate_up.shape[1] // 2


def silu_and_mul(gate_up, *, out=None):
    """bf16 [rows, 2W] (gate | up) -> bf16 [rows, W] = bf16(silu(gate) * up) (gk_silu_and_mul_bf16_v1)."""
    device = require_device(gate_up.device)
    rows, width = _check_gate_up(gate_up, device)
    if out is None:
        out = torch.empty((rows, width), dtype=torch.bfloat16, device=device)
    elif out.dtype != torch.bfloat16 or out.shape != (rows, width) or out.stride(1) != 1 or out.device != device:
        raise ValueError("out must be bf16 [rows, W] with unit column stride on the same GPU")
    nat.check("gk_silu_and_mul_bf16",
              nat.load().gk_silu_and_mul_bf16(_ptr(gate_up), rows, width, gate_up.stride(0), _ptr(out),
                                              out.stride(0), _stream(device)))
    return out


def silu_mul_quant(gate_up, *, native_half=False, m_pad=None, decode_layout=False):
    """SiLU-and-mul fused with the 1x128 quantizer -> (codes [G, m_pad, 128], sa [G, m_pad]) as act_quant
    of silu_and_mul(gate_up) would give; decode_layout as in act_quant."""
    device = require_device(gate_up.device)
    rows, width = _check_gate_up(gate_up, device)
    g = (width + 127) // 128
    m_pad = (16 * decode_tiles(rows) if decode_layout else rows) if m_pad is None else m_pad
    q = torch.empty((g, m_pad, 128), dtype=torch.uint8, device=device)
    sa = torch.empty((g, m_pad), dtype=torch.float32, device=device)
    flags = (nat.GK_FLAG_NATIVE_HALF if native_half else 0) | (nat.GK_FLAG_DECODE_LAYOUT if decode_layout else 0)
    nat.check("gk_fp8_silu_mul_quant_bf16",
              nat.load().gk_fp8_silu_mul_quant_bf16(_ptr(gate_up), rows, width, gate_up.stride(0), _ptr(q),
                                                    _ptr(sa), m_pad, flags, _stream(device)))
    return q, sa


def gelu_and_mul(gate_up, *, approximate=False, out=None):
    """bf16 [rows, 2W] (gate | up) -> bf16 [rows, W] = bf16(gelu(gate) * up) (gk_gelu_and_mul_bf16_v1);
    approximate=True is the tanh form."""
    device = require_device(gate_up.device)
    rows, width = _check_gate_up(gate_up, device)
    if out is None:
        out = torch.empty((rows, width), dtype=torch.bfloat16, device=device)
    elif out.dtype != torch.bfloat16 or out.shape != (rows, width) or out.stride(1) != 1 or out.device != device:
        raise ValueError("out must be bf16 [rows, W] with unit column stride on the same GPU")
    nat.check("gk_gelu_and_mul_bf16",
              nat.load().gk_gelu_and_mul_bf16(_ptr(gate_up), rows, width, gate_up.stride(0), _ptr(out),
                                              out.stride(0), int(bool(approximate)), _stream(device)))
    return out


def gelu_mul_quant(gate_up, *, approximate=False, native_half=False, m_pad=None, decode_layout=False):
    """GELU-and-mul fused with the 1x128 quantizer -> (codes [G, m_pad, 128], sa [G, m_pad]) as act_quant
    of gelu_and_mul(gate_up) would give; decode_layout as in act_quant."""
    device = require_device(gate_up.device)
    rows, width = _check_gate_up(gate_up, device)
    g = (width + 127) // 128
    m_pad = (16 * decode_tiles(rows) if decode_layout else rows) if m_pad is None else m_pad
    q = torch.empty((g, m_pad, 128), dtype=torch.uint8, device=device)
    sa = torch.empty((g, m_pad), dtype=torch.float32, device=device)
    flags = (nat.GK_FLAG_NATIVE_HALF if native_half else 0) | (nat.GK_FLAG_DECODE_LAYOUT if decode_layout else 0)
    nat.check("gk_fp8_gelu_mul_quant_bf16",
              nat.load().gk_fp8_gelu_mul_quant_bf16(_ptr(gate_up), rows, width, gate_up.stride(0),
                                                    int(bool(approximate)), _ptr(q), _ptr(sa), m_pad, flags,
                                                    _stream(device)))
    return q, sa


def _check_rows(t, name, device, width=None):
    if t.dtype != torch.bfloat16 or t.ndim != 2 or t.stride(1) != 1 or t.device != device:
        raise ValueError(f"{name} must be a 2-D bf16 tensor with unit column stride on the GPU")
    if width is not None and t.shape[1] != width:
        raise ValueError(f"{name} must have {width} columns")


def _norm_inputs(x, gamma, residual):
    device = require_device(x.device)
    _check_rows(x, "x", device)
    rows, width = x.shape
    if gamma.dtype != torch.bfloat16 or gamma.shape != (width,) or gamma.stride(0) != 1 or gamma.device != device:
        raise ValueError("gamma must be a contiguous bf16 [width] tensor on the same GPU")
    if residual is not None:
        _check_rows(residual, "residual", device, width)
        if residual.shape[0] != rows or residual.stride(0) != x.stride(0):
            raise ValueError("residual must have the shape and row stride of x")
    return device, rows, width


def rms_norm(x, gamma, epsilon=1e-6, weight_offset=0.0, *, out=None):
    """bf16 [rows, W] -> bf16 [rows, W] = bf16((x * inv) * (gamma + weight_offset)),
    inv = 1 / sqrt(mean(x^2) + epsilon) per row (gk_rms_norm_bf16_v1)."""
    device, rows, width = _norm_inputs(x, gamma, None)
    if out is None:
        out = torch.empty((rows, width), dtype=torch.bfloat16, device=device)
    else:
        _check_rows(out, "out", device, width)
    nat.check("gk_rms_norm_bf16",
              nat.load().gk_rms_norm_bf16(_ptr(x), rows, width, x.stride(0), _ptr(gamma), epsilon, weight_offset,
                                          _ptr(out), out.stride(0), _stream(device)))
    return out


def fused_add_rms_norm(x, residual, gamma, epsilon=1e-6, weight_offset=0.0):
    """-> (residual_out = bf16(x + residual), norm_out = rms_norm(residual_out)) (gk_fused_add_rms_norm_bf16_v1)."""
    device, rows, width = _norm_inputs(x, gamma, residual)
    res_out = torch.empty((rows, width), dtype=torch.bfloat16, device=device)
    norm_out = torch.empty((rows, width), dtype=torch.bfloat16, device=device)
    nat.check("gk_fused_add_rms_norm_bf16",
              nat.load().gk_fused_add_rms_norm_bf16(_ptr(x), _ptr(residual), rows, width, x.stride(0), _ptr(gamma),
                                                    epsilon, weight_offset, _ptr(res_out), _ptr(norm_out),
                                                    width, _stream(device)))
    return res_out, norm_out


def rms_norm_quant(x, gamma, epsilon=1e-6, weight_offset=0.0, *, residual=None, native_half=False, m_pad=None,
                   decode_layout=False):
    """(Fused add +) RMSNorm fused with the 1x128 quantizer -> (codes [G, m_pad, 128], sa [G, m_pad]) as
    act_quant of the normalized rows would give, plus residual_out (bf16 [rows, W]) when `residual` is given:
    (q, sa) or (q, sa, residual_out).  decode_layout as in act_quant."""
    device, rows, width = _norm_inputs(x, gamma, residual)
    g = (width + 127) // 128
    m_pad = (16 * decode_tiles(rows) if decode_layout else rows) if m_pad is None else m_pad
    q = torch.empty((g, m_pad, 128), dtype=torch.uint8, device=device)
    sa = torch.empty((g, m_pad), dtype=torch.float32, device=device)
    res_out = None if residual is None else torch.empty((rows, width), dtype=torch.bfloat16, device=device)
    flags = (nat.GK_FLAG_NATIVE_HALF if native_half else 0) | (nat.GK_FLAG_DECODE_LAYOUT if decode_layout else 0)
    nat.check("gk_fp8_rms_norm_quant_bf16",
              nat.load().gk_fp8_rms_norm_quant_bf16(_ptr(x), None if residual is None else _ptr(residual), rows,
                                                    width, x.stride(0), _ptr(gamma), epsilon, weight_offset,
                                                    None if res_out is None else _ptr(res_out), width, _ptr(q),
                                                    _ptr(sa), m_pad, flags, _stream(device)))
    return (q, sa) if residual is None else (q, sa, res_out)


def moe_rows_max(tokens, n_experts, top_k=2):
    """Padded row count of the expert-sorted layout (an upper bound of the rows in use)."""
    rows = ctypes.c_int64(0)
    nat.check("gk_fp8_moe_rows_max", nat.load().gk_fp8_moe_rows_max(tokens, n_experts, top_k, ctypes.byref(rows)))
    return rows.value


def moe_workspace_bytes(tokens, hidden, inter, n_experts, top_k=2):
    nbytes = ctypes.c_size_t(0)
    nat.check("gk_fp8_moe_workspace_bytes",
              nat.load().gk_fp8_moe_workspace_bytes(tokens, hidden, inter, n_experts, top_k, ctypes.byref(nbytes)))
    return nbytes.value


def moe_route(logits, top_k=2):
    """GPU routing -> (ids int32 [T, k], weights fp32 [T, k], row_of int32 [T, k], row_token int32 [R],
    offsets int32 [E + 1]); R = moe_rows_max(T, E, k), rows past offsets[E] are unused (-1)."""
    device = require_device(logits.device)
    if logits.dtype != torch.float32 or logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError("expected 2-D fp32 router logits [T, E] with unit column stride")
    t, e = logits.shape
    rows = moe_rows_max(t, e, top_k)
    ids = torch.empty((t, top_k), dtype=torch.int32, device=device)
    wts = torch.empty((t, top_k), dtype=torch.float32, device=device)
    row_of = torch.empty((t, top_k), dtype=torch.int32, device=device)
    row_token = torch.empty(rows, dtype=torch.int32, device=device)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=device)
    nat.check("gk_fp8_moe_route",
              nat.load().gk_fp8_moe_route(_ptr(logits), t, e, logits.stride(0), top_k, _ptr(ids), _ptr(wts),
                                          _ptr(row_of), _ptr(row_token), rows, _ptr(offsets), _stream(device)))
    return ids, wts, row_of, row_token, offsets


def moe_block_fp8(x, logits, w_gate_up, s_gate_up, w_down, s_down, *, top_k=2, native_half=False, out=None,
                  workspace=None):
    """Block-FP8 MoE layer: route, gather, gate_up GEMM, SiLU-and-mul, down GEMM, weighted combine.

    x bf16 [T, H]; logits fp32 [T, E]; w_gate_up E4M3 [E, 2I, H] (gate rows first), s_gate_up fp32
    [E, 2I/128, H/128]; w_down E4M3 [E, H, I], s_down fp32 [E, H/128, I/128] -> bf16 [T, H].
    Both expert weights may instead be pack_experts outputs (bit-identical results).
    """
    device = require_device(x.device)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("expected a 2-D bf16 activation with unit column stride")
    if logits.dtype != torch.float32 or logits.ndim != 2 or logits.stride(1) != 1 or logits.shape[0] != x.shape[0]:
        raise ValueError("expected fp32 router logits [T, E] with unit column stride")
    t, h = x.shape
    e = logits.shape[1]
    packed = isinstance(w_gate_up, PackedExperts)
    if packed != isinstance(w_down, PackedExperts):
        raise ValueError("pack both expert weights (pack_experts) or neither")
    for wt in (w_gate_up, w_down):
        if packed:
            if wt.data.dtype != torch.uint8 or wt.data.numel() < wt.e * packed_weight_bytes(wt.n, wt.k):
                raise ValueError("PackedExperts data is not a pack_experts output")
        elif wt.dtype not in (torch.float8_e4m3fn, torch.uint8) or wt.ndim != 3 or not wt.is_contiguous():
            raise ValueError("expected contiguous E4M3 expert weights [E, N, K]")
    inter = w_gate_up.shape[1] // 2
    if w_gate_up.shape != (e, 2 * inter, h) or w_down.shape != (e, h, inter):
        raise ValueError("expert weight shapes must be [E, 2I, H] and [E, H, I]")
    if (s_gate_up.shape != (e, (2 * inter + 127) // 128, (h + 127) // 128)
            or s_down.shape != (e, (h + 127) // 128, (inter + 127) // 128)):
        raise ValueError("expert scale shapes must be [E, 2I/128, H/128] and [E, H/128, I/128]")
    for tt in (logits, w_gate_up, s_gate_up, w_down, s_down):
        if tt.device != device:
            raise ValueError("all operands must be on the same GPU")
    for st in (s_gate_up, s_down):
        if st.dtype != torch.float32 or not st.is_contiguous():
            raise ValueError("expected contiguous fp32 expert scales")
    nbytes = moe_workspace_bytes(t, h, inter, e, top_k)
    ws = _checked_workspace(workspace, nbytes, device)
    if out is None:
        out = torch.empty((t, h), dtype=torch.bfloat16, device=device)
    elif out.dtype != torch.bfloat16 or out.shape != (t, h) or out.stride(1) != 1 or out.device != device:
        raise ValueError("out must be bf16 [T, H] with unit column stride on the same GPU")
    nat.check("gk_fp8_moe_bf16",
              nat.load().gk_fp8_moe_bf16(_ptr(x), t, h, x.stride(0), _ptr(logits), e, logits.stride(0), top_k,
                                         _ptr(w_gate_up.data if packed else _u8(w_gate_up)), _ptr(s_gate_up),
                                         inter, _ptr(w_down.data if packed else _u8(w_down)), _ptr(s_down),
                                         _ptr(out), out.stride(0),
                                         (nat.GK_FLAG_NATIVE_HALF if native_half else 0)
                                         | (nat.GK_FLAG_WEIGHT_PACKED if packed else 0), _ptr(ws), ws.numel(),
                                         _stream(device)))
    return out


def weights_finite(weight, scales):
    """True iff the E4M3FN weight holds no NaN code and its scales are finite and >= 0 (GPU check)."""
    x = torch.zeros((1, weight.shape[-1]), dtype=torch.bfloat16, device=weight.device)
    return inputs_finite(x, weight.reshape(-1, weight.shape[-1]), scales)


def token_quant(x, *, out=None, scales=None):
    """Per-token W8A8 activation quantization (gk_fp8_token_quant_bf16_v1) -> (half-range codes uint8
    [rows, width], scales fp32 [rows] = 2 * max|x_row| / 448)."""
    device = require_device(x.device)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("expected a 2-D bf16 activation with unit column stride")
    rows, width = x.shape
    q = torch.empty((rows, width), dtype=torch.uint8, device=device) if out is None else out
    s = torch.empty(rows, dtype=torch.float32, device=device) if scales is None else scales
    nat.check("gk_fp8_token_quant_bf16",
              nat.load().gk_fp8_token_quant_bf16(_ptr(x), rows, width, x.stride(0), _ptr(q), q.stride(0), _ptr(s),
                                                 _stream(device)))
    return q, s


def channel_finish(partial, act_scales, w_scales, bias=None, *, out=None):
    """y = bf16(fma(partial * act_scales[:, None], w_scales, bias)) (gk_fp8_channel_finish_bf16_v1)."""
    device = require_device(partial.device)
    rows, width = partial.shape
    y = torch.empty((rows, width), dtype=torch.bfloat16, device=device) if out is None else out
    nat.check("gk_fp8_channel_finish_bf16",
              nat.load().gk_fp8_channel_finish_bf16(_ptr(partial), rows, width, partial.stride(0), _ptr(act_scales),
                                                    _ptr(w_scales), _ptr(bias), _ptr(y), y.stride(0),
                                                    _stream(device)))
    return y


def channel_gemm(q, sa, weight, sw, bias=None, *, out=None):
    """Per-token / per-channel W8A8 GEMM: codes q [M, K] with sa [M], weight codes [N, K] with sw [N] ->
    bf16 [M, N] = bf16(fma(sum_k q w * sa, sw, bias))."""
    device = require_device(q.device)
    q8, w8 = _u8(q), _u8(weight)
    m, k = q8.shape
    n = w8.shape[0]
    if w8.shape[1] != k or not w8.is_contiguous() or q8.stride(1) != 1:
        raise ValueError("expected codes q [M, K] (unit column stride) and a contiguous weight [N, K]")
    if sa.shape != (m,) or sw.shape != (n,) or (bias is not None and bias.shape != (n,)):
        raise ValueError("expected sa [M], sw [N] and bias [N]")
    y = torch.empty((m, n), dtype=torch.bfloat16, device=device) if out is None else out
    nat.check("gk_fp8_channel_gemm_bf16",
              nat.load().gk_fp8_channel_gemm_bf16(_ptr(q8), q8.stride(0), _ptr(sa), m, k, _ptr(w8), n, _ptr(sw),
                                                  _ptr(bias), _ptr(y), y.stride(0), 0, _stream(device)))
    return y


def token_channel_fused_pays(m, n, k):
    """Whether the one-launch form (gk_fp8_token_channel_gemm_bf16, up to 16 rows) beats token_quant +
    channel_gemm.  Every workgroup of the fused form reads its rows' whole activation twice (the token
    maximum, then the codes), so it pays only for few rows and little redundant work, measured on MI355X
    (one launch / two): N = 6144, K = 4096: 8.7 / 9.2 us at M <= 4, 10.4 / 10.0 at M = 8; N = 4096,
    K = 14336: 16.1 / 19.1 us at M <= 4, 22.7 / 19.5 at M = 8; N = 28672, K = 4096: 24.4 / 23.4 us."""
    return m <= 4 and (-(-n // 32) / 256) * (k / 4096) <= 2.0


def token_channel_gemm(x, weight, sw, bias=None, *, out=None, fused=None):
    """Per-token / per-channel W8A8 on bf16 activations: token_quant then channel_gemm, or both in one
    launch (gk_fp8_token_channel_gemm_bf16, bit-identical) where token_channel_fused_pays (fused=None) or
    when fused=True (up to 16 rows; x 16-byte aligned with a row stride that is a multiple of 8)."""
    device = require_device(x.device)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("expected a 2-D bf16 activation with unit column stride")
    m, k = x.shape
    n = _u8(weight).shape[0]
    if fused is None:
        fused = token_channel_fused_pays(m, n, k)
    fused = fused and m <= 16 and x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0
    if not fused:
        q, sa = token_quant(x)
        return channel_gemm(q, sa, weight, sw, bias, out=out)
    w8 = _u8(weight)
    if w8.shape[1] != k or not w8.is_contiguous():
        raise ValueError("expected a contiguous weight [N, K]")
    if sw.shape != (n,) or (bias is not None and bias.shape != (n,)):
        raise ValueError("expected sw [N] and bias [N]")
    y = torch.empty((m, n), dtype=torch.bfloat16, device=device) if out is None else out
    nat.check("gk_fp8_token_channel_gemm_bf16",
              nat.load().gk_fp8_token_channel_gemm_bf16(_ptr(x), x.stride(0), m, k, _ptr(w8), n, _ptr(sw),
                                                        _ptr(bias), _ptr(y), y.stride(0), 0, _stream(device)))
    return y


# ---- K ranges and the row-parallel completion ---------------------------------------------


def block_fp8_gemm_kslice(x, weight, scales, k_offset, k_len, *, native_half=False, variant=None, out=None,
                          accumulate=False, workspace=None):
    """fp32 partial of the block-FP8 GEMM over the K columns [k_offset, k_offset + k_len) (asynchronous).

    x bf16 [M, K], weight [N, K] (row-major codes or a PackedWeight), scales the whole
    [ceil(N/128), K/128] grid.  Returns out fp32 [M, N] (allocated when None) holding
    sum_g P_g * sa * sw over the range's groups, added to out's contents when accumulate=True
    (the reference's chunked prefill chain carries c0 over K chunks this way,
    fp8_hybrid_tpcsim_test.cpp:253-302).  k_offset and k_len: multiples of 128 inside K
    (generic_fp8_glue.hpp:169-176, :245-252).  variant: None, "decode" or "prefill".
    """
    device = require_device(x.device)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.stride(1) != 1:
        raise ValueError("expected a 2-D bf16 activation with unit column stride")
    _check_gemm_operands(weight, scales, None, device)
    m, k = x.shape
    w8, n, kw, wflag = _weight_args(weight)
    if kw != k:
        raise ValueError("activation and weight K differ")
    if variant == "generic":
        raise ValueError("the K-range GEMM runs the decode or the LDS-tiled variant")
    flags = _flags(native_half, variant) | wflag
    _, _, ws_bytes = plan(m, n, max(128, int(k_len)), flags, w8)
    ws = _checked_workspace(workspace, ws_bytes, device)
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs the partial to add to (out)")
        out = torch.empty((m, n), dtype=torch.float32, device=device)
    elif out.dtype != torch.float32 or out.shape != (m, n) or out.stride(1) != 1 or out.device != device:
        raise ValueError("out must be fp32 [M, N] with unit column stride on the same GPU")
    if accumulate:
        flags |= nat.GK_FLAG_ACCUMULATE
    lib = nat.load()
    nat.check("gk_fp8_block_gemm_kslice_f32",
              lib.gk_fp8_block_gemm_kslice_f32(_ptr(x), m, k, x.stride(0), int(k_offset), int(k_len), _ptr(w8), n,
                                               _ptr(scales), scales.shape[0], scales.shape[1], _ptr(out),
                                               out.stride(0), flags, _ptr(ws), ws.numel(), _stream(device)))
    return out


def partial_finish(partial, bias=None, *, out=None):
    """bf16(partial + bias) of an fp32 partial [rows, width] (the decode reduce's last step, reduce_bias.c:42-57)."""
    device = require_device(partial.device)
    if partial.dtype != torch.float32 or partial.ndim != 2 or partial.stride(1) != 1:
        raise ValueError("expected a 2-D fp32 partial with unit column stride")
    rows, width = partial.shape
    if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous() or bias.numel() != width
                             or bias.device != device):
        raise ValueError("expected a contiguous fp32 bias with `width` elements on the same GPU")
    if out is None:
        out = torch.empty((rows, width), dtype=torch.bfloat16, device=device)
    elif (out.dtype != torch.bfloat16 or out.ndim != 2 or tuple(out.shape) != (rows, width) or out.stride(1) != 1
          or out.device != device):
        raise ValueError("out must be a bf16 [rows, width] tensor with unit column stride on the partial's GPU")
    lib = nat.load()
    nat.check("gk_fp8_partial_finish_bf16",
              lib.gk_fp8_partial_finish_bf16(_ptr(partial), rows, width, partial.stride(0), _ptr(bias), _ptr(out),
                                             out.stride(0), _stream(device)))
    return out


def rank_sum_infer(gathered_elems, world_size):
    """Slice length of a gathered buffer (infer_rank_sum, generic_dense_glue.cpp:871-895)."""
    elems = ctypes.c_int64(0)
    nat.check("gk_rank_sum_infer", nat.load().gk_rank_sum_infer(int(gathered_elems), int(world_size),
                                                                 ctypes.byref(elems)))
    return elems.value


def rank_sum(gathered, world_size, *, out=None):
    """Ordered sum of world_size contiguous slices of a 1-D fp32 or bf16 buffer (rank_sum.c:4-42).

    gathered: [world_size * elems] (what an all-gather of the ranks' slices leaves).  Returns
    [elems] of the same dtype: ((s_0 + s_1) + s_2) + ... in fp32, one bf16 rounding for bf16.
    """
    device = require_device(gathered.device)
    if gathered.ndim != 1 or not gathered.is_contiguous() or gathered.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("expected a contiguous 1-D fp32 or bf16 gathered buffer")
    elems = rank_sum_infer(gathered.numel(), world_size)
    if out is None:
        out = torch.empty(elems, dtype=gathered.dtype, device=device)
    elif out.dtype != gathered.dtype or out.numel() != elems or not out.is_contiguous() or out.device != device:
        raise ValueError("out must be a contiguous [elems] buffer of the gathered dtype")
    lib = nat.load()
    fn = lib.gk_rank_sum_f32 if gathered.dtype == torch.float32 else lib.gk_rank_sum_bf16
    nat.check(fn.__name__, fn(_ptr(gathered), gathered.numel(), int(world_size), _ptr(out), elems,
                              _stream(device)))
    return out
