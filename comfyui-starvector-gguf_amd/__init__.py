"""MI355X (gfx950) implementation of the quantized GGUF GEMV path of
ComfyUI-StarVector-GGUF: `quantization` mirrors the reference's quantized-op
module on top of the HIP library libsvq.so; `decoder` holds the
StarCoder2/GPTBigCode-style decode harness that drives it."""
