"""Graph data: partitioning, adjacency plans, GCN normalisation, synthetic inputs."""
