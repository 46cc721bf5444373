"""Mutation check of the oracle's pinning tests.

Each mutant plants one plausible mistake in a copy of oracle/npa_oracle.c (a dropped term, a
flipped sign, a wrong exponent, index or loop order, a broken hash constant, an unstable sort),
builds it with the oracle's own flags and runs tests/test_oracle.py against it through
NPA_ORACLE_LIB. Every mutant must make that suite fail: a mistake that no pinning test notices
would leave the oracle - and so every GPU parity claim that rests on it - unchecked.
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "npa_oracle.c")
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-shared"]

# name -> (text in npa_oracle.c, replacement); the text must occur in the source
MUTANTS = {
    "radius_not_strict": ("if (r2 < eps2) nbuf_push", "if (r2 <= eps2) nbuf_push"),
    "cell_walk_dx_outer": (
        "for (int dy = -1; dy <= 1; ++dy)\n            for (int dx = -1; dx <= 1; ++dx) {\n"
        "                int64_t coords[3] = {center[0] + dx",
        "for (int dx = -1; dx <= 1; ++dx)\n            for (int dy = -1; dy <= 1; ++dy) {\n"
        "                int64_t coords[3] = {center[0] + dx"),
    "delta_sign": ("float v = rhs[a] - lhs[a];", "float v = lhs[a] - rhs[a];"),
    "unstable_bins": ("uint32_t dst = counts[bin]++;",
                      "uint32_t dst = bin_offsets[bin + 1] - 1 - (counts[bin]++ - bin_offsets[bin]);"),
    "mix_multiplier": ("x *= 0x7feb352du;", "x *= 0x7feb352fu;"),
    "poly6_exponent": ("4.0f / (PI_F * powi_f32(cfg->eps, 8))", "4.0f / (PI_F * powi_f32(cfg->eps, 6))"),
    "spiky_cubed": ("3.0f * (t * t) / r;", "3.0f * (t * t * t) / r;"),
    "blur_volume_dropped": ("blur_row[c] += sj[c] * smooth * volume_j;", "blur_row[c] += sj[c] * smooth;"),
    "gradient_diff_sign": ("float diff = sj[c] - si[c];\n                    for (uint32_t a = 0; a < d; ++a) grad_row",
                           "float diff = si[c] - sj[c];\n                    for (uint32_t a = 0; a < d; ++a) grad_row"),
    "moment_uncorrected": ("pg[c * d + k] * inv[k * d + o]", "pg[c * d + k] * (k == o ? 1.0f : 0.0f)"),
    "density_grad_power": ("powi_f32(cfg->eps / eps0, 1 + (int)cfg->dim)", "powi_f32(cfg->eps / eps0, (int)cfg->dim)"),
    "log1p_as_log": ("float scale = log1pf(norm) / norm;", "float scale = logf(1.0f + norm) / norm;"),
    "mlp_bias_dropped": ("float sum = w->b1[h];", "float sum = 0.0f;"),
    "relu_dropped": ("hidden[h] = fmaxf(sum, 0.0f);", "hidden[h] = sum;"),
    "motion_norm_squared": ("meps / (1.0f + norm);", "meps / (1.0f + norm * norm);"),
    "state_mask_ignored": ("float next = s[c] + dt * dsr[c] * m;", "float next = s[c] + dt * dsr[c];"),
    "mem_dims_3d": ("return cfg->dim == 3 ? 4 : 2;", "return cfg->dim == 3 ? 3 : 2;"),
    "clamp_channel": ("(c == 3 || (S > 8 && c == 8))", "(c == 4 || (S > 8 && c == 8))"),
    "mask_hash_multiplier": ("x = x * 0x27d4eb2du;", "x = x * 0x27d4eb2fu;"),
    "decode_colour_offset": ("clamp_f32(s[base + ch] + 0.5f, 0.0f, 1.0f);", "clamp_f32(s[base + ch] + 0.4f, 0.0f, 1.0f);"),
    "splat_radius": ("ceilf(5.0f * sigma)", "ceilf(3.0f * sigma)"),
    "iso_up": ("b[3] = {1.0f, 1.0f, 2.0f}", "b[3] = {1.0f, 1.0f, 1.0f}"),
    "xz_swapped": ("case NPA_VIEW_XZ: r = I[0], u = I[2], f = I[1];", "case NPA_VIEW_XZ: r = I[0], u = I[1], f = I[2];"),
    "depth_unhalved": ("0.5f + 0.5f * render_dot3(p, fwd)", "0.5f + render_dot3(p, fwd)"),
    "render_y_not_flipped": ("float py = (ws - pp[1])", "float py = (ws + pp[1])"),
    "render_sigma2": ("/ (2.0f * sigma2));", "/ sigma2);"),
    "render_radius": ("fmaxf(ceilf(5.0f * sigma), 1.0f)", "fmaxf(ceilf(4.0f * sigma), 1.0f)"),
    "render_count_norm": ("const float norm_scale = 1.0f / (float)(count > 1 ? count : 1);",
                          "const float norm_scale = 1.0f;"),
    "render_opacity_dropped": ("wbuf[k] / denom * norm_scale * opacity;", "wbuf[k] / denom * norm_scale;"),
    "render_depth_channel": ("px5[4] += pp[2] * w;", "px5[4] += pp[1] * w;"),
    "render_sigma_unclamped": ("fmaxf(clamp_f32(sigmas[n], cfg->min_sigma, cfg->max_sigma), RENDER_EPS)",
                               "fmaxf(sigmas[n], RENDER_EPS)"),
    "opacity_channel": ("S > 8 ? 8 : (S > 3 ? 3 : -1)", "S > 8 ? 7 : (S > 3 ? 3 : -1)"),
    "sigmoid_sign": ("return 1.0f / (1.0f + expf(-v));", "return 1.0f / (1.0f + expf(v));"),
    "adj_poly6_factor": ("out[a] = out_adj * dk * 2.0f * delta[a];", "out[a] = out_adj * dk * delta[a];"),
    "adj_spiky_radial": ("out[a] = scale * out_adj[a] + dscale_dr * dot * delta[a] / r;", "out[a] = scale * out_adj[a];"),
    "adj_log_radial": ("in_adj[k] += scale * out_adj[k] + radial * in[k];", "in_adj[k] += scale * out_adj[k];"),
    "adj_volume_sign": ("density_adj[j] -= v_adj / (rho * rho);", "density_adj[j] += v_adj / (rho * rho);"),
    "adj_position_sign": ("pos_adj[4 * lhs + a] -= d_adj[a];", "pos_adj[4 * lhs + a] += d_adj[a];"),
    # (transposing either factor is no mistake: the inverse and the moment matrix are symmetric)
    "adj_inverse_adjoint_sign": ("            m_adj[row * d + col] -= v;", "            m_adj[row * d + col] += v;"),
    "adj_self_gradient": ("state_adj[idx * S + c] -= sc;", "(void)sc;"),
    "adj_blur_weight": ("state_adj[(uint64_t)n->j * S + c] += badj[c] * w;", "state_adj[(uint64_t)n->j * S + c] += badj[c] * kern;"),
    "adj_density_kernel_pass": ("poly6_delta_adjoint(n->delta, n->r2, cfg, adj, da);", "poly6_delta_adjoint(n->delta, n->r2, cfg, 0.0f, da);"),
    "adj_hybrid_grad": ("gda[cc] += a * n->delta[r];", "gda[cc] += 0.0f * n->delta[r];"),
    "adj_dgrad_scale": ("for (uint32_t a = 0; a < d; ++a) radj[a] *= scale;\n            } else {",
                        "for (uint32_t a = 0; a < d; ++a) radj[a] *= 1.0f;\n            } else {"),
    "render_learned_channel": ("float logit = clamp_f32(s[S - 5]", "float logit = clamp_f32(s[S - 4]"),
    "decode_learned_channel": ("float scale_logit = clamp_f32(s[S - 5]", "float scale_logit = clamp_f32(s[S - 6]"),
    "decode_opacity_channel": ("float opacity_logit = clamp_f32(s[S - 4]", "float opacity_logit = clamp_f32(s[S - 5]"),
    "raster_lowpass_dropped": ('U[0][2] * T[0][2]) + 0.3f;', 'U[0][2] * T[0][2]);'),
    "raster_y_not_flipped": ('const float tx = vx, ty = -vy, tz = -vz;', 'const float tx = vx, ty = vy, tz = -vz;'),
    "raster_conic_cross_sign": ('out->qb = (-b / det) * -L;', 'out->qb = (b / det) * -L;'),
    "raster_power_cross_sign": ('fmaf(g->qc * dy, dy, g->qb * dx * dy)', 'fmaf(g->qc * dy, dy, -g->qb * dx * dy)'),
    "raster_log2e_dropped": ('out->qa = (c / det) * (-0.5f * L);', 'out->qa = (c / det) * -0.5f;'),
    "raster_alpha_clamp": ('fminf(0.99f, g->opacity * exp2f(p2))', 'fminf(1.0f, g->opacity * exp2f(p2))'),
    "raster_alpha_floor": ('if (alpha < 1.0f / 255.0f) continue;', 'if (alpha < 1.0f / 64.0f) continue;'),
    "raster_no_cut": ('if (next < 0.0001f) break;', 'if (next < 0.0f) break;'),
    "raster_pixel_centre": ('const float pxc = (float)px + 0.5f,', 'const float pxc = (float)px,'),
    "raster_back_to_front": ('if (da < db) return -1;\n    if (da > db) return 1;', 'if (da < db) return 1;\n    if (da > db) return -1;'),
    "raster_tie_order": ('return ia < ib ? -1 : (ia > ib ? 1 : 0);', 'return ia > ib ? -1 : (ia < ib ? 1 : 0);'),
    "raster_quat_transposed": ('2.0f * (qx * qy - qw * qz), 2.0f * (qx * qz + qw * qy)}', '2.0f * (qx * qy + qw * qz), 2.0f * (qx * qz - qw * qy)}'),
    "raster_scale_row": ('M[r][c] = R[r][c] * so[c];', 'M[r][c] = R[r][c] * so[r];'),
    "raster_radius": ('const float radius = ceilf(3.0f * sqrtf(lam));', 'const float radius = ceilf(2.0f * sqrtf(lam));'),
    "raster_sh1_sign": ('basis[1] = -kShC1 * y;', 'basis[1] = kShC1 * y;'),
    "raster_sh2_term": ('basis[6] = kShC2[2] * (2.0f * zz - xx - yy);', 'basis[6] = kShC2[2] * (2.0f * zz - xx + yy);'),
    "raster_sh3_term": ('kShC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);', 'kShC3[3] * z * (2.0f * zz - 3.0f * xx - 2.0f * yy);'),
    "raster_sh_offset": ('        acc += 0.5f;\n        out[ch]', '        acc += 0.25f;\n        out[ch]'),
    "raster_view_dir_sign": ('float d[3] = {pv[0] - campos[0], pv[1] - campos[1], pv[2] - campos[2]};', 'float d[3] = {campos[0] - pv[0], campos[1] - pv[1], campos[2] - pv[2]};'),
    "export_tail_order": ("export_tail_channel(s, S, 2), export_tail_channel(s, S, 1),\n                               export_tail_channel(s, S, 0)",
                          "export_tail_channel(s, S, 0), export_tail_channel(s, S, 1),\n                               export_tail_channel(s, S, 2)"),
    "export_sh_offset": ("c[ch] = (color - 0.5f) / ORACLE_SH_C0;", "c[ch] = color / ORACLE_SH_C0;"),
    "export_iso_scale": ("fmaxf(eps * 0.12f, 0.00008f);", "fmaxf(eps * 0.1f, 0.00008f);"),
    "export_quat_sign": ("const float q[4] = {1.0f + u[2], -u[1], u[0], 0.0f};",
                         "const float q[4] = {1.0f + u[2], u[1], u[0], 0.0f};"),
    "export_density_scale": ("sqrtf(4096.0f / fmaxf((float)particle_count, 1.0f))",
                             "sqrtf(1024.0f / fmaxf((float)particle_count, 1.0f))"),
    "export_tangent_z": ("scale[2] = fmaxf(tangent * 0.18f, 0.00008f);", "scale[2] = fmaxf(tangent * 0.5f, 0.00008f);"),
    "export_opacity_channel": ("export_channel(s, S, S > 8 ? 8u : 3u);", "export_channel(s, S, S > 8 ? 7u : 3u);"),
    "export_2d_z": ("pv[2] = dim == 3 ? p[2] : 0.0f;", "pv[2] = p[2];"),
    "raster_camera_centre": ('out[k] = -(V[k] * V[3] + V[4 + k] * V[7] + V[8 + k] * V[11]);', 'out[k] = -(V[4 * k] * V[3] + V[4 * k + 1] * V[7] + V[4 * k + 2] * V[11]);'),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistake_is_caught(name, tmp_path):
    old, new = MUTANTS[name]
    src = open(SRC).read()
    assert old in src, f"mutation site of {name} no longer in the oracle source"
    mutant = tmp_path / "npa_oracle_mutant.c"
    mutant.write_text(src.replace(old, new, 1))
    lib = tmp_path / "libnpa_oracle_mutant.so"
    subprocess.run(["gcc", *CFLAGS, "-I", os.path.join(ROOT, "oracle"), "-I",
                    os.path.join(ROOT, "include"), "-o", str(lib), str(mutant), "-lm"], check=True)
    env = dict(os.environ, NPA_ORACLE_LIB=str(lib), OMP_NUM_THREADS="2")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_oracle.py")], cwd=ROOT, env=env,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    assert r.returncode == 1, f"mutant {name} survived the pinning tests:\n{r.stdout[-2000:]}"
