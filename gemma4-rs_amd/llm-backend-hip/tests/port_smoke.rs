//! `HipPort` against the known answers of the CPU backend's tests
//! (crates/llm-backend-cpu/tests/ops_smoke.rs) and its error texts; the
//! device KV cache's `ContextMemory` errors (context_memory.rs:53-69); and
//! `attend` against a plain loop.  Needs an MI355X (device 0):
//! `cargo test -p llm-backend-hip`.

use llm_backend_hip::{DeviceKvCache, HipPort};
use llm_eng::compute::ComputePort;
use llm_eng::EngError;

fn port() -> HipPort {
    HipPort::new(0).expect("a HIP device")
}

fn compute_text(err: EngError) -> String {
    match err {
        EngError::Compute(text) => text,
        other => panic!("expected EngError::Compute, got {other:?}"),
    }
}

#[test]
fn port_matmul_2x2() {
    // ops_smoke.rs:16-24 and 112-122
    let p = port();
    let a = p.upload(&[1.0, 2.0, 3.0, 4.0]).unwrap();
    let b = p.upload(&[5.0, 6.0, 7.0, 8.0]).unwrap();
    let c = p.matmul(&a, &b, 2, 2, 2).unwrap();
    assert_eq!(p.download(&c).unwrap(), vec![19.0, 22.0, 43.0, 50.0]);
}

#[test]
fn port_rms_norm_scales_unit_vector() {
    // ops_smoke.rs:34-43
    let p = port();
    let x = p.upload(&[3.0, 4.0]).unwrap();
    let w = p.upload(&[1.0, 1.0]).unwrap();
    let y = p.download(&p.rms_norm(&x, &w, 0.0).unwrap()).unwrap();
    assert!((y[0] - 0.848_528_15).abs() < 1e-6);
    assert!((y[1] - 1.131_370_9).abs() < 1e-6);
}

#[test]
fn port_elementwise_ops_and_rope_rotate_pairs() {
    // ops_smoke.rs:84-99
    let p = port();
    let a = p.upload(&[1.0, 2.0]).unwrap();
    let b = p.upload(&[3.0, 4.0]).unwrap();
    assert_eq!(p.download(&p.add(&a, &b).unwrap()).unwrap(), vec![4.0, 6.0]);
    let s = p.download(&p.softmax(&a).unwrap()).unwrap();
    assert!((s[0] - 0.268_941_43).abs() < 1e-6);
    assert!((s[1] - 0.731_058_6).abs() < 1e-6);
    let mut v = p.upload(&[1.0, 0.0]).unwrap();
    p.rope(&mut v, 1, 1.0, 2).unwrap();
    let v = p.download(&v).unwrap();
    assert!((v[0] - 1.0_f32.cos()).abs() < 1e-6);
    assert!((v[1] - 1.0_f32.sin()).abs() < 1e-6);
}

#[test]
fn port_errors_carry_the_cpu_texts() {
    let p = port();
    let two = p.upload(&[1.0, 2.0]).unwrap();
    let three = p.upload(&[1.0, 2.0, 3.0]).unwrap();
    let empty = p.upload(&[]).unwrap();
    assert_eq!(compute_text(p.matmul(&two, &two, 2, 2, 2).unwrap_err()), "matmul buffer shape does not match dimensions");
    assert_eq!(compute_text(p.matmul(&two, &two, usize::MAX, 2, 2).unwrap_err()), "matmul dimensions overflow");
    assert_eq!(compute_text(p.add(&two, &three).unwrap_err()), "add buffer lengths differ");
    assert_eq!(compute_text(p.rms_norm(&two, &three, 0.0).unwrap_err()), "invalid RMS norm inputs");
    assert_eq!(compute_text(p.rms_norm(&two, &two, -1.0).unwrap_err()), "invalid RMS norm inputs");
    assert_eq!(compute_text(p.softmax(&empty).unwrap_err()), "softmax requires a non-empty buffer");
    let nan = p.upload(&[1.0, f32::NAN]).unwrap();
    assert_eq!(compute_text(p.softmax(&nan).unwrap_err()), "softmax input is not finite");
    let mut x = p.upload(&[1.0, 2.0]).unwrap();
    assert_eq!(compute_text(p.rope(&mut x, 1, 1.0, 3).unwrap_err()), "invalid RoPE inputs");
    assert_eq!(compute_text(p.rope(&mut x, 1, 0.0, 2).unwrap_err()), "invalid RoPE inputs");
}

#[test]
fn kv_cache_views_report_the_reference_errors() {
    let p = port();
    let mut cache = DeviceKvCache::new(&p, &[4, 4], 8).unwrap();
    let k = p.upload(&[1.0; 8]).unwrap();
    let v = p.upload(&[2.0; 8]).unwrap();
    cache.append_rows(&p, 0, &k, &v, 2).unwrap();
    assert_eq!(cache.len(0), 2);
    assert_eq!(cache.view(0, 2).unwrap().len(), 2);
    // context_memory.rs:62-67: more rows than appended
    match cache.view(0, 3) {
        Err(EngError::ContextTooLong { got: 3, max: 2 }) => {}
        other => panic!("{other:?}"),
    }
    // context_memory.rs:54-60: a layer never appended to, len > 0
    match cache.view(1, 1) {
        Err(EngError::MissingLayer(1)) => {}
        other => panic!("{other:?}"),
    }
    assert!(cache.view(1, 0).unwrap().is_empty());
    cache.clear();
    assert_eq!(cache.len(0), 0);
}

#[test]
fn attend_matches_a_plain_loop() {
    let p = port();
    let (n_heads, n_kv_heads, head_dim, t) = (8usize, 1usize, 256usize, 37usize);
    let value = |i: usize, salt: usize| (((i * 7919 + salt * 104_729) % 1000) as f32 / 500.0) - 1.0;
    let q: Vec<f32> = (0..n_heads * head_dim).map(|i| value(i, 1)).collect();
    let keys: Vec<Vec<f32>> = (0..t).map(|r| (0..head_dim).map(|i| value(i + r * head_dim, 2)).collect()).collect();
    let values: Vec<Vec<f32>> = (0..t).map(|r| (0..head_dim).map(|i| value(i + r * head_dim, 3)).collect()).collect();
    let got = p.attend(&q, &keys, &values, n_heads, n_kv_heads, 1.0).unwrap();
    for h in 0..n_heads {
        let qh = &q[h * head_dim..(h + 1) * head_dim];
        let scores: Vec<f64> =
            keys.iter().map(|k| qh.iter().zip(k).map(|(a, b)| f64::from(*a) * f64::from(*b)).sum()).collect();
        let max = scores.iter().cloned().fold(f64::NEG_INFINITY, f64::max);
        let weights: Vec<f64> = scores.iter().map(|s| (s - max).exp()).collect();
        let total: f64 = weights.iter().sum();
        for d in 0..head_dim {
            let want: f64 = weights.iter().zip(&values).map(|(w, v)| w / total * f64::from(v[d])).sum();
            assert!((f64::from(got[h * head_dim + d]) - want).abs() < 1e-4, "head {h} dim {d}");
        }
    }
    assert_eq!(compute_text(p.attend(&q, &[], &[], n_heads, n_kv_heads, 1.0).unwrap_err()), "softmax input is not finite");
}
