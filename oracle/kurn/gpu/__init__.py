"""kurn.gpu (restated subset): `ref`, the reference problem generators and exact references."""
