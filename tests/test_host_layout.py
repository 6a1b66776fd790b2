"""Host-side layer layout of the decoder (no GPU): Gemma-4-E2B's per-layer
head dims, FFN widths and KV producer map (src/config/gemma4-e2b.ts:16-63 and
159-180, src/types.ts:79-91), and the uniform benchmark layout."""
from g4hip.decoder import E2BShape


def test_real_layout_follows_the_e2b_config():
    s = E2BShape.real()
    glob = (4, 9, 14, 19, 24, 29, 34)
    assert s.global_layers == glob and s.n_layers == 35
    # consumers read the last unshared layer of their kind: 13 (local), 14 (global)
    assert [s.producer(i) for i in range(35)] == list(range(15)) + [14 if i in glob else 13 for i in range(15, 35)]
    assert [s.is_producer(i) for i in range(35)] == [i < 15 for i in range(35)]
    assert [s.hd(i) for i in range(35)] == [512 if i in glob else 256 for i in range(35)]
    assert [s.ffn_of(i) for i in range(35)] == [6144 if i < 15 else 12288 for i in range(35)]
    assert s.q_dim == 4096 and s.kv_dim == 512 and s.max_ffn == 12288
    assert s.q_dim_of(4) == 4096 and s.q_dim_of(3) == 2048


def test_real_layout_weight_bytes():
    """Per-layer matrix bytes: Q4_K (144 B per 256) q/k/v/o/gate/up, Q6_K
    (210 B per 256) down; consumers carry no k/v projections."""
    s = E2BShape.real()
    H = 1536

    def layer(hd, ffn, kv):
        q4 = (8 * hd * H * 2 + (2 * hd * H if kv else 0) + 2 * ffn * H) // 256 * 144
        return q4 + H * ffn // 256 * 210

    assert s.layer_weight_bytes(0) == layer(256, 6144, True)
    assert s.layer_weight_bytes(4) == layer(512, 6144, True)
    assert s.layer_weight_bytes(15) == layer(256, 12288, False)
    assert s.layer_weight_bytes(19) == layer(512, 12288, False)
    assert s.weight_bytes() == sum(layer(s.hd(i), s.ffn_of(i), i < 15) for i in range(35))


def test_uniform_layout_is_unchanged():
    s = E2BShape()
    assert all(s.producer(i) == i for i in range(35))
    assert all(s.hd(i) == 256 and s.ffn_of(i) == 6144 for i in range(35))
    assert s.q_dim == 2048 and s.kv_dim == 256
    small = E2BShape.real(n_layers=6, n_unshared=3, global_layers=(1, 4))
    assert [small.producer(i) for i in range(6)] == [0, 1, 2, 2, 1, 2]
