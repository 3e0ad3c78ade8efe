"""Model configuration (field names and meaning of model/config.py:7-48)."""

from dataclasses import dataclass


@dataclass
class ModelConfig:
    # architecture
    vocab_size: int = 32000
    n_layer: int = 12
    n_embd: int = 768
    n_head: int = 12
    n_kv_head: int = 4
    head_dim: int = 64
    ffn_dim: int = 2048

    # forecast
    forecast_heads: int = 4
    forecast_dim: int = 64

    # context / positions
    context_length: int = 1024
    rope_theta: float = 10000.0

    # regularisation / init
    norm_eps: float = 1e-6
    tie_embeddings: bool = True
    initializer_range: float = 0.02

    # attention backend: "hip_sparse" (aliases "sparse", "forecast", ...),
    # "static_sparse", "hip_async_offload"
    attention_backend: str = "hip_sparse"
    sparse_mode: str = "forecast"

    # block routing
    block_size: int = 32
    top_k_blocks: int = 4
    num_queries_per_kv: int = 3

    # Decode routing of the HIP backend: "reference" scores the forecast with
    # the causal mask at query row 0 exactly as model/attention/sparse.py:139
    # does (only block 0 competes; the remaining picks are the lowest-index
    # -inf ties), "absolute" masks at the query's true position.
    decode_routing: str = "reference"

    # HIP model only: compute RMSNorm + the q / k / v / forecast projections +
    # RoPE of each block in one kernel (sparda.produce) when the attention
    # backend is one of the HIP ones and the activations are bf16.
    fused_producer: bool = False

    # HIP model only: for decode-sized batches (B*T <= 16 rows, bf16, no
    # autograd) compute ffn_norm + SwiGLU + the residual add of each block in
    # two kernels (sparda.ffn_decode).
    fused_ffn: bool = False

    def __post_init__(self):
        if self.n_head * self.head_dim != self.n_embd:
            raise AssertionError(f"{self.n_head} query heads of dim {self.head_dim} do not tile "
                                 f"the {self.n_embd}-wide residual stream")
        if self.n_head % self.n_kv_head:
            raise AssertionError(f"{self.n_kv_head} key/value heads cannot be shared evenly by "
                                 f"{self.n_head} query heads")
        if self.decode_routing not in ("reference", "absolute"):
            raise AssertionError(f"unknown decode_routing {self.decode_routing!r} "
                                 "(expected 'reference' or 'absolute')")
        self.num_queries_per_kv = self.n_head // self.n_kv_head
