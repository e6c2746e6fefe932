# A dense layer whose flat loops run the batch fastest (the products' outputs transposed
# against the weights' storage): a test text of the lowering's contractions
# (tests/test_lower_contract.py, tests/test_gpu_contract.py).
function dense_b(y, x, xb, w, wb, i_b, i_in, i_h)
    for idx = 1:i_h * i_b
        i_j = div(idx - 1, i_b) + 1
        i_s = mod(idx - 1, i_b) + 1
        s = 0.0
        for i_k = 1:i_in
            s = s + x[(i_k - 1) * i_b + i_s] * w[(i_k - 1) * i_h + i_j]
        end
        y[idx] = s
    end
    for idx = i_h * i_b:-1:1
        i_j = div(idx - 1, i_b) + 1
        i_s = mod(idx - 1, i_b) + 1
        sb = y[idx] + 1.0
        for i_k = 1:i_in
            wb[(i_k - 1) * i_h + i_j] = wb[(i_k - 1) * i_h + i_j] + sb * x[(i_k - 1) * i_b + i_s]
            xb[(i_k - 1) * i_b + i_s] = xb[(i_k - 1) * i_b + i_s] + w[(i_k - 1) * i_h + i_j] * sb
        end
    end
    return nothing
end
