"""bench.py may use the CPU oracle only in its CPU-baseline leg: every `from oracle import ...` /
`import oracle` statement in bench.py must sit inside an `if do_cpu:` block, so a run with --no-cpu
never loads the oracle.  The product package itself must not import it at all."""
import ast
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _oracle_imports(tree):
    for node in ast.walk(tree):
        if isinstance(node, ast.ImportFrom) and (node.module or "").split(".")[0] == "oracle":
            yield node
        elif isinstance(node, ast.Import) and any(a.name.split(".")[0] == "oracle" for a in node.names):
            yield node


def _inside_do_cpu(tree, target):
    """True if `target` is nested in the body of an `if` whose test mentions the name do_cpu."""
    def walk(node, guarded):
        if node is target:
            return guarded
        for child in ast.iter_child_nodes(node):
            g = guarded
            if isinstance(node, ast.If) and child in node.body:
                g = guarded or any(isinstance(n, ast.Name) and n.id == "do_cpu" for n in ast.walk(node.test))
            r = walk(child, g)
            if r is not None:
                return r
        return None
    return bool(walk(tree, False))


def test_bench_imports_oracle_only_in_cpu_leg():
    with open(os.path.join(ROOT, "bench.py")) as f:
        tree = ast.parse(f.read())
    imports = list(_oracle_imports(tree))
    assert imports, "bench.py's CPU-baseline leg is expected to use the oracle"
    for node in imports:
        assert _inside_do_cpu(tree, node), f"bench.py:{node.lineno} imports the oracle outside an `if do_cpu:` block"


def test_package_never_imports_oracle():
    pkg = os.path.join(ROOT, "vernondsl_amd")
    for name in sorted(os.listdir(pkg)):
        if name.endswith(".py"):
            with open(os.path.join(pkg, name)) as f:
                tree = ast.parse(f.read())
            assert not list(_oracle_imports(tree)), f"vernondsl_amd/{name} imports the oracle"
