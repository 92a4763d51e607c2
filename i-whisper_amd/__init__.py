"""MI355X (gfx950) integer I-Whisper encoder/decoder path.

Layer API mirroring the reference's i_whisper/model_int.py and
i_whisper/modules/linear.py, backed by hand-written HIP kernels reached through
the C ABI in include/iwhisper_amd.h.
"""
from . import _lib, kernels, synth  # noqa: F401
from .linear import Linear8, Linear32, LinearBase, set_linear8_backend, set_linear32_backend  # noqa: F401
from .model_int import (  # noqa: F401
    AudioEncoder_int, Conv1d_int, GELU_int, LayerNorm_int, ModelDimensions, MultiHeadAttention_int,
    ResidualAttentionBlock_int, TextDecoder_int, Whisper_int, set_all_backends,
    set_attention_backend, set_conv1d_backend, set_decoder_backend, set_encoder_backend,
    set_gelu_backend, set_layernorm_backend, set_residual_backend)
from .runtime import DecoderRunner, EncoderRunner, GreedyResult, LogitFilters, greedy_decode  # noqa: F401
from . import audio, checkpoint, timing  # noqa: F401
from .checkpoint import (  # noqa: F401
    load_int_model, load_int_params, save_int_model, verify_int_model_roundtrip)

# Whisper model shapes (n_mels, n_audio_ctx, d, heads, layers, vocab, n_text_ctx)
SHAPES = {
    "tiny": ModelDimensions(80, 1500, 384, 4, 4, 51865, 448, 384, 4, 4),  # 4 heads as the CPU case
    "base": ModelDimensions(80, 1500, 512, 8, 6, 51865, 448, 512, 8, 6),
    "small": ModelDimensions(80, 1500, 768, 12, 12, 51865, 448, 768, 12, 12),
    "medium": ModelDimensions(80, 1500, 1024, 16, 24, 51865, 448, 1024, 16, 24),
    "large": ModelDimensions(128, 1500, 1280, 20, 32, 51865, 448, 1280, 20, 32),
}
