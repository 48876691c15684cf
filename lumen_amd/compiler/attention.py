"""Flash-attention matching (``lumen/graph_compiler/passes/attention/``) — filled in below."""


def match(graph):
    return graph


def lower(plan, step):
    raise NotImplementedError("flash attention: the hip backend has no kernel for it yet")
