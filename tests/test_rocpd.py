"""k3moe.rocpd's summaries on small synthetic rocpd databases (CPU)."""

import sqlite3

from k3moe import rocpd


def make_db(path, rows, counters):
    con = sqlite3.connect(path)
    con.execute('create table kernels (name text, lds_size int, duration int, start int)')
    con.execute('create table counters_collection (dispatch_id int, counter_name text, kernel_name text, '
                'lds_block_size int, grid_size int, value real, start int)')
    con.executemany('insert into kernels values (?, ?, ?, ?)', rows)
    con.executemany('insert into counters_collection values (?, ?, ?, ?, ?, ?, ?)', counters)
    con.commit()
    con.close()


def test_kernel_table_groups_by_kernel_and_lds(tmp_path):
    kt = tmp_path / 'kt.db'
    make_db(kt, [('void k3moe::k_latent<0>(k3moe::LatPlan)', 100, 20000, 1),
                 ('void k3moe::k_latent<0>(k3moe::LatPlan)', 100, 22000, 2),
                 ('k3moe::k_moe_single(k3moe::Plan)', 200, 15000, 3),
                 ('void k3moe::k_latent<0>(k3moe::LatPlan)', 300, 30000, 4)], [])
    fe = tmp_path / 'fe.db'
    make_db(fe, [], [(1, 'FETCH_SIZE', '__amd_rocclr_copyBuffer', 0, 1, 512.0, 0),
                     (2, 'FETCH_SIZE', 'void k3moe::k_latent<0>(k3moe::LatPlan)', 100, 1, 10.0, 1),
                     (2, 'FETCH_SIZE', 'void k3moe::k_latent<0>(k3moe::LatPlan)', 100, 1, 6.0, 1),
                     (3, 'FETCH_SIZE', 'k3moe::k_moe_single(k3moe::Plan)', 200, 1, 4.0, 2)])
    rows = rocpd.kernel_table(str(kt), str(fe), None, ['k_latent', 'k_moe'], 1024 * 1024)
    assert [(r['kernel'], r['lds_bytes'], r['dispatches']) for r in rows] == [
        ('k_latent<0>', 100, 2), ('k_moe_single', 200, 1), ('k_latent<0>', 300, 1)]
    assert rows[0]['median_us'] == 21.0 and rows[0]['avg_us'] == 21.0
    # the copy probe reported 512 units for 1 MiB: 2048 bytes per unit; dispatch 2 summed 16 units
    assert rows[0]['read_bytes'] == 16 * 2048 and rows[1]['read_bytes'] == 4 * 2048
    assert 'read_bytes' not in rows[2] and 'write_bytes' not in rows[0]
