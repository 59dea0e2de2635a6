"""MI355X-native drop-in for Wayfinder's fused causal top-K + sparse attention path.

Mirrors the import paths of the reference package ``routing_attention`` for that path
only: ``routing_attention.kernels`` (causal_topk, sparse_meat_attention,
fused_sparse_attention), ``routing_attention.models`` (the learned-address, key-vector and routing sparse
attention modules, their address/router projections and the TransformerLM decoder around
them) and ``routing_attention.retrieval`` (RetrievalConfig, RoutingRetriever).
"""
