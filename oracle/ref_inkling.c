/* ref_inkling.c -- the Inkling engine's own MoE layer, moe() (c/inkling.c:1011-1185),
 * on host weights: c/inkling.c compiled where it lies with main() renamed, and a
 * Model / Layer set up around one sparse layer whose routed experts all sit in
 * that layer's expert cache as packed int4 container slots (the state the
 * engine's cache reaches once every expert has been filled, so moe() takes
 * cache hits only and reads no disk).  The shared experts are bf16 residents,
 * which moe() runs through matmul_h.
 *
 * TEST INFRASTRUCTURE ONLY (oracle/_ref): pins the oracle's Inkling routing and
 * gated shared experts to the engine's real code path.  The routed experts'
 * matmul contract is the engine's matmul_q4, which reads IDOT from the
 * environment once per process (IDOT=0: the f32 route). */
#define main inkling_main_unused
#include "inkling.c"
#undef main

/* out[S,D] = moe(x[S,D]) of layer 0: E routed experts of per-row int4 (gu_q
 * [E*2I, D/2], gu_s [E*2I], dn_q [E*D, I/2], dn_s [E*D]), an f32 router
 * [E+ns, D] with its correction bias [E], ns bf16 shared experts ([ns*I, D],
 * [ns*I, D], [ns*D, I]); route_scale and the gate's global_scale as the
 * engine holds them. */
int ref_inkling_moe(int E, int K, int ns, float route_scale, float gscale, int D, int I,
                    const float *router, const float *rbias,
                    const uint8_t *gu_q, const float *gu_s, const uint8_t *dn_q, const float *dn_s,
                    const uint16_t *sg, const uint16_t *su, const uint16_t *sd,
                    const float *x, float *out, int S) {
    static Model m;
    static Layer L;
    static LCache lc;
    memset(&m, 0, sizeof m); memset(&L, 0, sizeof L); memset(&lc, 0, sizeof lc);
    m.c.hidden = D; m.c.n_experts = E; m.c.topk = K; m.c.n_shared = ns; m.c.moe_inter = I;
    m.c.route_scale = route_scale;
    m.xq = 1; m.rb13 = D / 2; m.rb2 = I / 2;        /* container int4: q4 = rb13 * 2 == D */
    Slot *slots = calloc((size_t)E, sizeof(Slot));
    if (!slots) return -1;
    for (int e = 0; e < E; e++) {
        slots[e].eid = e; slots[e].filled = 1;
        slots[e].p13 = (uint8_t *)gu_q + (size_t)e * 2 * I * (D / 2);
        slots[e].s13 = (float *)gu_s + (size_t)e * 2 * I;
        slots[e].p2 = (uint8_t *)dn_q + (size_t)e * D * (I / 2);
        slots[e].s2 = (float *)dn_s + (size_t)e * D;
    }
    lc.slots = slots; lc.n = E; lc.cap = E;
    m.cache = &lc;
    uint32_t *eusage[1] = {NULL};
    uint8_t *seen[1] = {NULL};
    int *prev_topm[1] = {NULL};
    m.eusage = eusage; m.seen = seen; m.prev_topm = prev_topm;
    L.router = (float *)router; L.rbias = (float *)rbias; L.rgs = gscale;
    L.sh_g.h = (uint16_t *)sg; L.sh_u.h = (uint16_t *)su; L.sh_d.h = (uint16_t *)sd;
    moe(&m, &L, 0, (float *)x, S, out);
    free(slots);
    return 0;
}
