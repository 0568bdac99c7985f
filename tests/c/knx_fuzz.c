/* knx_fuzz.c — loader fuzz harness, built by tests/test_fuzz.py with AddressSanitizer and UBSan over the host
 * runtime sources.  Every file named on the command line is loaded; a file the loader accepts must describe a
 * consistent model (checked below, all on the host: no forward runs here) and is freed again.  A memory error or
 * undefined behaviour aborts the process; an inconsistent accepted model exits with status 3.
 * Output: "accepted <n> of <m>". */
#include <stdio.h>
#include <stdlib.h>

#include "kernix_model.h"

/* the invariants every loaded model keeps: sizes positive and within int, values in range, the output value last
 * read at the end, every input of a step an earlier value, storage buffers inside the planned region */
static int consistent(const kernix_model* m)
{
    if (m->n_steps < 1 || m->in_dim < 1 || m->out_dim < 1 || m->seq_len < 1 || m->n_vals != m->n_steps + 1) return 0;
    if (m->out_v < 0 || m->out_v >= m->n_vals || m->vals[m->out_v].last != m->n_steps) return 0;
    for (int i = 0; i < m->n_steps; i++) {
        const kernix_step* s = &m->steps[i];
        if (s->kind < 0 || s->kind > KERNIX_OP_LAST || s->n_in < 1 || s->n_in > KERNIX_MAX_INPUTS) return 0;
        for (int k = 0; k < s->n_in; k++)
            if (s->inp[k] < 0 || s->inp[k] > i) return 0;
    }
    for (int v = 0; v < m->n_vals; v++) {
        const kernix_val* x = &m->vals[v];
        if (x->nd < 1 || x->nd > KERNIX_MAX_DIMS || x->r < 1 || x->c < 1) return 0;
        if (x->st >= m->n_st) return 0;
        if (x->st >= 0 && m->st_off[x->st] + (size_t)x->r * (size_t)x->c > m->st_span) return 0;
    }
    return 1;
}

int main(int argc, char** argv)
{
    int accepted = 0;
    for (int i = 1; i < argc; i++) {
        kernix_model* m = kernix_model_load(argv[i]);
        if (m == NULL) continue;
        accepted++;
        if (!consistent(m)) {
            fprintf(stderr, "inconsistent model accepted: %s\n", argv[i]);
            return 3;
        }
        kernix_model_free(m);
    }
    printf("accepted %d of %d\n", accepted, argc - 1);
    return 0;
}
