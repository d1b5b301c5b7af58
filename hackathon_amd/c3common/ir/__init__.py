from .graph import Edge, Graph, Node, ONNSType, Tensor, generate_node_id

__all__ = ["Edge", "Graph", "Node", "ONNSType", "Tensor", "generate_node_id"]
