from routing_attention.retrieval.index import (
    RetrievalConfig,
    RoutingRetriever,
    retrieval_config_from_dict,
)

__all__ = ["RetrievalConfig", "RoutingRetriever", "retrieval_config_from_dict"]
